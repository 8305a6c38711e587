// Device-side helpers shared by the qw35 HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace qw35 {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// DPP controls (GCN/CDNA encoding).
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;
constexpr int kDppRowRor4 = 0x124;      // row_ror:4 (within each 16-lane row)
constexpr int kDppRowRor8 = 0x128;      // row_ror:8

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the 64 lanes of a wave; the total is valid in lane 63.
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
    v += dpp_f32<kDppQuadXor1>(v);
    v += dpp_f32<kDppQuadXor2>(v);
    v += dpp_f32<kDppRowHalfMirror>(v);
    v += dpp_f32<kDppRowMirror>(v);
    v += dpp_f32<kDppRowBcast15, 0xA>(v);
    v += dpp_f32<kDppRowBcast31, 0xC>(v);
    return v;
}

// Sum over the 64 lanes, broadcast to every lane (through lane 63).
__device__ __forceinline__ float wave_sum(float v) {
    v = wave_sum_to_lane63(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v, uint32_t moved) { return v > moved ? v : moved; }

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, false);
}

// max |v| over the 64 lanes, broadcast.  |v| is compared as its bit pattern
// (ordered like the value for non-NaN; a NaN lane makes the result NaN), with
// 0 as the identity so each step is one DPP-modified v_max_u32.
__device__ __forceinline__ float wave_max_abs(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v) & 0x7FFFFFFFu;
    u = dpp_max_u32(u, dpp_u32<kDppQuadXor1>(u));
    u = dpp_max_u32(u, dpp_u32<kDppQuadXor2>(u));
    u = dpp_max_u32(u, dpp_u32<kDppRowHalfMirror>(u));
    u = dpp_max_u32(u, dpp_u32<kDppRowMirror>(u));
    u = dpp_max_u32(u, dpp_u32<kDppRowBcast15, 0xA>(u));
    u = dpp_max_u32(u, dpp_u32<kDppRowBcast31, 0xC>(u));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane((int)u, 63));
}

// Lanes l and l ^ 16 (v_permlane16_swap), l and l ^ 32 (v_permlane32_swap):
// the larger of the two values in both.
__device__ __forceinline__ uint32_t max_xor16_u32(uint32_t v) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return dpp_max_u32(p[0], p[1]);
}
__device__ __forceinline__ uint32_t max_xor32_u32(uint32_t v) {
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return dpp_max_u32(p[0], p[1]);
}

// Wave maxima of NB rows at once (NB = 1, 2, 4, 8): m[r] is lane's value of
// row r (non-negative fp32 bit patterns, compared as integers); returns the
// maximum of row r over the 64 lanes in out[r] (uniform).
// The first log2(NB) steps each halve the rows a lane carries: at the step on
// lane bit j a lane keeps the half of its rows selected by its bit j, merged
// with the same rows of its partner across that bit (row_ror:4 for bit 2,
// quad permutations for bits 1 and 0).  Lane l is then left with row l % NB
// over the lanes that agree with it outside those bits, and the remaining
// steps (one value each) pair lanes that agree on those bits.  8 rows cost 28
// VALU operations instead of 48 for eight separate reductions.
template <int NB>
__device__ __forceinline__ void wave_max_rows(const uint32_t (&m)[NB], uint32_t (&out)[NB], int lane) {
    static_assert(NB == 1 || NB == 2 || NB == 4 || NB == 8, "NB");
    uint32_t a[NB];
#pragma unroll
    for (int r = 0; r < NB; ++r) a[r] = m[r];
    auto halve = [&](auto CTRL, int held, bool upper) {
        constexpr int ctrl = decltype(CTRL)::value;
#pragma unroll
        for (int r = 0; r < NB / 2; ++r) {
            if (r < held / 2) {
                const uint32_t lo = dpp_max_u32(a[r], dpp_u32<ctrl>(a[r]));
                const uint32_t hi = dpp_max_u32(a[r + held / 2], dpp_u32<ctrl>(a[r + held / 2]));
                a[r] = upper ? hi : lo;
            }
        }
    };
    if constexpr (NB == 8) halve(std::integral_constant<int, kDppRowRor4>{}, 8, (lane & 4) != 0);
    if constexpr (NB >= 4) halve(std::integral_constant<int, kDppQuadXor2>{}, 4, (lane & 2) != 0);
    if constexpr (NB >= 2) halve(std::integral_constant<int, kDppQuadXor1>{}, 2, (lane & 1) != 0);
    uint32_t u = a[0];
    if constexpr (NB == 1) u = dpp_max_u32(u, dpp_u32<kDppQuadXor1>(u));
    if constexpr (NB <= 2) u = dpp_max_u32(u, dpp_u32<kDppQuadXor2>(u));
    if constexpr (NB <= 4) u = dpp_max_u32(u, dpp_u32<kDppRowRor4>(u));
    u = dpp_max_u32(u, dpp_u32<kDppRowRor8>(u));
    u = max_xor16_u32(u);
    u = max_xor32_u32(u);
#pragma unroll
    for (int r = 0; r < NB; ++r) out[r] = (uint32_t)__builtin_amdgcn_readlane((int)u, r);
}

__device__ __forceinline__ float dot2(half2_t a, half2_t b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
}

__device__ __forceinline__ half2_t as_half2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// v as a materialised fp32 value: the empty asm keeps the compiler from fusing
// the fma that produced v with a following fp16 conversion into v_fma_mix,
// whose single rounding straight to fp16 differs from fp16(fl32(x)) whenever
// the fp32 rounding of x is inexact.
__device__ __forceinline__ float keep_f32(float v) {
    asm("" : "+v"(v));
    return v;
}

// fp32 -> fp16 round-to-nearest-even, packed.
__device__ __forceinline__ half2_t h2(float lo, float hi) {
    half2_t r;
    r.x = (_Float16)lo;
    r.y = (_Float16)hi;
    return r;
}

// Streaming 16-byte load of weights that are read exactly once.
__device__ __forceinline__ uint4_t load_stream16(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint4_t*>(p));
}

// Cached 16-byte load of weights whose 128-byte lines are read again soon by
// other waves: prefill weight tiles (every token tile of the launch reads
// them) and k-quant chunks that do not end on a line boundary (the next
// chunk's wave reads the rest of the line).  A streaming load lets L2 drop
// such a line before its second reader arrives.
__device__ __forceinline__ uint4_t load_cached16(const void* p) {
    return *reinterpret_cast<const uint4_t*>(p);
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

// Power-of-two factor 2^e that brings max_abs into [2^13, 2^14), so that every
// scaled activation fits fp16 (max 65504) with headroom and the small ones stay
// clear of fp16 subnormals; 1 for zero, inf or NaN input.  |e| <= 125 covers
// every finite fp32 maximum down to 2^-111 exactly (smaller maxima land below
// 2^13, still normal in fp16 down to 2^-139), and keeps 2^(e+1) -- the prefill
// staging doubles the factor -- and its inverse normal fp32 numbers.
__device__ __forceinline__ float fp16_range_scale(float max_abs) {
    if (!(max_abs > 0.0f) || !(max_abs <= 3.4028234663852886e38f)) return 1.0f;
    int e;
    (void)frexpf(max_abs, &e);  // max_abs in [2^(e-1), 2^e)
    int shift = 14 - e;         // max_abs * 2^shift < 2^14
    if (shift > 125) shift = 125;
    if (shift < -125) shift = -125;
    return ldexpf(1.0f, shift);
}

// fp16_range_scale and its inverse from the bit pattern of max_abs (a
// non-negative fp32 or an inf/NaN pattern), in integer operations, so that a
// uniform maximum is scaled on the scalar unit.  For a normal maximum with
// biased exponent E the factor is 2^(140 - E); subnormal maxima (E = 0) and
// everything below 2^-111 take 2^125.
__device__ __forceinline__ void fp16_range_scale_bits(uint32_t max_bits, float& sc, float& inv) {
    if (max_bits == 0u || max_bits >= 0x7F800000u) {
        sc = 1.0f;
        inv = 1.0f;
        return;
    }
    int shift = 140 - (int)(max_bits >> 23);
    shift = shift < 125 ? shift : 125;
    sc = __builtin_bit_cast(float, (uint32_t)(127 + shift) << 23);
    inv = __builtin_bit_cast(float, (uint32_t)(127 - shift) << 23);
}

// 1 / s for s = 2^e, |e| <= 126 (fp16_range_scale returns |e| <= 125, the
// prefill staging at most 2^126): the exponent field is mirrored about 127,
// so the result is exact.
__device__ __forceinline__ float pow2_inverse(float s) {
    return __builtin_bit_cast(float, 0x7F000000u - __builtin_bit_cast(uint32_t, s));
}

}  // namespace qw35
