// Shared definitions for the gfx950 routed-MoE-experts kernels.
//
// Conventions used across the kernels:
//   T tokens, H hidden, F expert intermediate, E experts, K top-k, P = T*K routed pairs.
//   A "pair" p = t*K + k is one (token, top-k slot) entry of top_k_index[T, K].
//   Pairs are grouped by expert in op_eager order: expert ascending, then slot k, then token t
//   (transformers Cohere2MoeExperts.forward: torch.where over the [K, T] one-hot slice,
//   modeling_cohere2_moe.py:122-130).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cmoe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// Word 3 of a raw buffer descriptor on gfx9-family GPUs (gfx950 included): 32-bit data format,
// no swizzle, no index stride. Loads past num_records return 0 without a memory access.
constexpr int kBufferWord3 = 0x00020000;

// Weight layouts (mirrors include/cernels_moe.h).
constexpr int kLayoutConcat = 0;       // gate_up [E, 2F, H] (gate rows, then up rows), down [E, H, F]
constexpr int kLayoutInterleaved = 1;  // gate_up [E, H, 2F] (even col gate, odd col up), down [E, F, H]
// Activations.
constexpr int kActSilu = 0;    // silu(gate) * up
constexpr int kActGptOss = 1;  // (clamp(up,-7,7) + 1) * g * sigmoid(1.702 g), g = min(gate, 7)
// Non-gated (one projection, h -> act(h)), megablocks_moe's act_id 0 / 1 / 2.
constexpr int kActGeluTanh = 2;  // 0.5 h (1 + tanh(sqrt(2/pi) (h + 0.044715 h^3)))
constexpr int kActSiluPlain = 3; // h sigmoid(h)
constexpr int kActRelu = 4;      // max(h, 0)
__host__ __device__ constexpr bool act_is_gated(int act) { return act == kActSilu || act == kActGptOss; }

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 bits (same rounding torch uses for .to(bfloat16)).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    __bf16 b = (__bf16)f;
    return __builtin_bit_cast(uint16_t, b);
}

// SwiGLU variants in fp32. The logistic factor 1/(1+exp(-x)) uses the hardware reciprocal
// (v_rcp_f32, about 1 ulp): the result is rounded to bf16 right after, so the division's last bits
// never reach the output.
//   silu:   transformers ACT2FN["silu"] = x * sigmoid(x)  (modeling_cohere2_moe.py:131)
//   gpt-oss: GptOssExperts._apply_gate (modeling_gpt_oss.py:82-88), alpha 1.702, limit 7.0
// The clamps are IEEE minimum/maximum (v_minimum3_f32 / v_maximum3_f32): a nan propagates, as through
// torch.clamp in the transformers module (fminf / fmaxf, as in src/kops/gpt_oss_moe_experts/csrc/
// gpt_oss_moe_experts.cu:98-99, would clamp it to a finite +-7).
template <int ACT>
__device__ __forceinline__ float swiglu(float gate, float up) {
    if constexpr (ACT == kActSilu) {
        return gate * __builtin_amdgcn_rcpf(1.0f + __expf(-gate)) * up;
    } else {
        gate = __builtin_elementwise_minimum(gate, 7.0f);
        up = __builtin_elementwise_minimum(__builtin_elementwise_maximum(up, -7.0f), 7.0f);
        const float glu = gate * __builtin_amdgcn_rcpf(1.0f + __expf(-1.702f * gate));
        return (up + 1.0f) * glu;
    }
}

// Non-gated activations in fp32 (src/kops/megablocks_moe/csrc/megablocks_moe.cu:78-96 lists the
// three). GELU's tanh form is Hendrycks & Gimpel's approximation; tanh(u) = 1 - 2 / (1 + e^{2u}),
// which saturates to +-1 through the exponential's overflow and underflow.
template <int ACT>
__device__ __forceinline__ float act_plain(float h) {
    if constexpr (ACT == kActGeluTanh) {
        const float u = 0.7978845608028654f * (h + 0.044715f * h * h * h);
        const float th = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + __expf(2.0f * u));
        return 0.5f * h * (1.0f + th);
    } else if constexpr (ACT == kActSiluPlain) {
        return h * __builtin_amdgcn_rcpf(1.0f + __expf(-h));
    } else {
        return __builtin_elementwise_maximum(h, 0.0f);  // a nan propagates, as through torch.relu
    }
}

// Two fp32 values -> two round-to-nearest-even bf16 in one dword (low half = a).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
}

// Two fp32 values -> two round-to-nearest-even fp16 in one dword (low half = a).
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}

// 24-bit floats: the top 24 bits of the fp32 pattern (sign, 8-bit exponent, 15-bit mantissa), rounded
// to nearest even on the 8 dropped bits (2^-16 relative rounding, fp32's range; values past the largest
// 24-bit float round to inf). inf stays inf; a nan becomes the quiet nan (its rounding could carry it
// into inf). Four values pack into three dwords, value i in bytes 3i..3i+2.
// f32_round24: the fp32 pattern with the rounding added, whose top 24 bits are the 24-bit float (the low
// byte is left over); four VALU instructions per value.
__device__ __forceinline__ uint32_t f32_round24(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t r = u + 0x7fu + ((u >> 8) & 1u);
    return __builtin_isnan(f) ? 0x7fc00000u : r;
}
__device__ __forceinline__ float f24_to_f32(uint32_t r) { return __uint_as_float(r << 8); }
struct f24x4 {
    uint32_t d[3];
};
// The three dwords are bytes 1..3 of the four rounded patterns in order, gathered with one v_perm_b32 each
// (byte k of the result is byte sel_k of {first operand : second operand}, 0..3 the second, 4..7 the first).
__device__ __forceinline__ f24x4 pack_f24x4(float a, float b, float c, float e) {
    const uint32_t r0 = f32_round24(a), r1 = f32_round24(b), r2 = f32_round24(c), r3 = f32_round24(e);
    return f24x4{{__builtin_amdgcn_perm(r1, r0, 0x05030201u), __builtin_amdgcn_perm(r2, r1, 0x06050302u),
                  __builtin_amdgcn_perm(r3, r2, 0x07060503u)}};
}
__device__ __forceinline__ f32x4 unpack_f24x4(const f24x4& p) {
    return f32x4{f24_to_f32(p.d[0] & 0xffffffu), f24_to_f32((p.d[0] >> 24) | ((p.d[1] & 0xffffu) << 8)),
                 f24_to_f32((p.d[1] >> 16) | ((p.d[2] & 0xffu) << 16)), f24_to_f32(p.d[2] >> 8)};
}

// Half-wave exchange (v_permlane32_swap_b32): lanes 32..63 of a and lanes 0..31 of b trade places, so lane l
// of a afterwards holds b's lane l - 32 (l >= 32) and lane l of b holds a's lane l + 32 (l < 32).
__device__ __forceinline__ void swap_halves(uint32_t& a, uint32_t& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}
// The larger of lane l's and lane l ^ 32's values, in both lanes (fmaxf: a nan is passed over).
__device__ __forceinline__ float max_halves(float v) {
    uint32_t a = __float_as_uint(v), b = a;
    swap_halves(a, b);
    return fmaxf(__uint_as_float(a), __uint_as_float(b));
}

// Full-wave (64-lane) maximum; every lane returns it.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Full-wave (64-lane) sum; every lane returns the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__host__ __device__ constexpr int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Per-XCD item ranges of the two packed GEMMs (gate_up g = 0, down g = 1), written by the route
// kernel once the expert histogram is known: XCD x of GEMM g takes items
// [bounds[9g + x], bounds[9g + x + 1]). Shapes of the two launches are fixed by the host beforehand.
struct XcdSplit {
    int fw[2];        // fragments per item
    int n_tiles[2];   // N-tiles (items per M-tile)
    int slots[2];     // workgroups per XCD
    int32_t* bounds;  // [2][9], or null: no split is written
};

}  // namespace cmoe
