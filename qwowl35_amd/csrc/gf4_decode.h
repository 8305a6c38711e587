// GF4 word -> exact fp16 MFMA operand (shared by the GF4 GEMV kernels).
//
// Word (GGUF type 100): bits 0..7 an e5m2 scale byte b (s = fp16(b << 8)), bits
// 8+3i..10+3i the code c_i = q_i ^ 4 of column 8g+i; the weight is
// (4 - q_i) * s / 4 (tools/qw35_cook_common.py:67-80,115-119).
//
// Word -> 8 exact fp16 weights, 15 VALU ops:
//   t1 = w >> 4, t2 = w >> 10
//   P0 = (t1 & 0x00070070) ^ M'A       fp16 pair (64 + q0, 1024 + q4)
//   P1 = (t1 & 0x00380380) ^ M'B       fp16 pair ( 8 + q1,  128 + q5)
//   P2 = (t2 & 0x00070070) ^ M'A       fp16 pair (64 + q2, 1024 + q6)
//   P3 = (t2 & 0x00380380) ^ M'B       fp16 pair ( 8 + q3,  128 + q7)
//   E_j = P_j * (-1/4) + (base + 4)/4 = (4 - q)/4     (exact)
//   B_j = E_j * s                                     (exact: 3 significant bits)
// where M' folds the code flip q = c ^ 4 into the magic constants.  The pairs
// hold columns (0,4) (1,5) (2,6) (3,7), so the activation operand is stored in
// the same order within each group of 8 columns.
#pragma once

#include "qw35_device.h"

namespace qw35 {

constexpr uint32_t kFlip = 0x92492400u;
constexpr uint32_t kMaskA = 0x00070070u;
constexpr uint32_t kMaskB = 0x00380380u;
constexpr uint32_t kMagicA = 0x64005400u;
constexpr uint32_t kMagicB = 0x58004800u;

// Loop-invariant operands of the decode, held in VGPRs so that the VOP3 forms
// (v_bitop3_b32, v_pk_fma_f16) take them without literals.
struct Gf4Consts {
    uint32_t mask_a, mask_b, magic_a, magic_b;
    half2_t quarter_neg, off_a, off_b;
};

// (t & mask) ^ magic' = ((t ^ flip) & mask) | magic: the code flip q = c ^ 4
// (bit 2 of every field) is folded into the magic constants.
constexpr uint32_t kMagicFlipA = kMagicA ^ ((kFlip >> 4) & kMaskA);  // == ((kFlip >> 10) & kMaskA) ^ kMagicA
constexpr uint32_t kMagicFlipB = kMagicB ^ ((kFlip >> 4) & kMaskB);
static_assert(((kFlip >> 4) & kMaskA) == ((kFlip >> 10) & kMaskA), "flip bits agree for both shifts");
static_assert(((kFlip >> 4) & kMaskB) == ((kFlip >> 10) & kMaskB), "flip bits agree for both shifts");

__device__ __forceinline__ Gf4Consts gf4_consts() {
    Gf4Consts c;
    c.mask_a = kMaskA;
    c.mask_b = kMaskB;
    c.magic_a = kMagicFlipA;
    c.magic_b = kMagicFlipB;
    c.quarter_neg = h2(-0.25f, -0.25f);
    c.off_a = h2(68.0f / 4.0f, 1028.0f / 4.0f);
    c.off_b = h2(12.0f / 4.0f, 132.0f / 4.0f);
    return c;
}

// v_bitop3_b32 with truth table 0x6a: (a & b) ^ c.
__device__ __forceinline__ uint32_t and_xor(uint32_t a, uint32_t mask, uint32_t bits) {
    return __builtin_amdgcn_bitop3_b32(a, mask, bits, 0x6a);
}

// One GF4 word -> MFMA B operand: 8 exact fp16 weights in column order
// 0,4,1,5,2,6,3,7 (15 VALU ops).
//   E_j = P_j * (-1/4) + (base + 4)/4 = (4 - q)/4   (exact)
//   B_j = E_j * s                                   (exact, |B| <= |s|)
__device__ __forceinline__ half8_t gf4_word_to_b(uint32_t w, const Gf4Consts& c) {
    const uint32_t t1 = w >> 4;
    const uint32_t t2 = w >> 10;
    const half2_t p0 = as_half2(and_xor(t1, c.mask_a, c.magic_a));
    const half2_t p1 = as_half2(and_xor(t1, c.mask_b, c.magic_b));
    const half2_t p2 = as_half2(and_xor(t2, c.mask_a, c.magic_a));
    const half2_t p3 = as_half2(and_xor(t2, c.mask_b, c.magic_b));
    const half2_t e0 = __builtin_elementwise_fma(p0, c.quarter_neg, c.off_a);
    const half2_t e1 = __builtin_elementwise_fma(p1, c.quarter_neg, c.off_b);
    const half2_t e2 = __builtin_elementwise_fma(p2, c.quarter_neg, c.off_a);
    const half2_t e3 = __builtin_elementwise_fma(p3, c.quarter_neg, c.off_b);
    // (b << 24) | (b << 8): the e5m2 byte as the high byte of both halves = (s, s).
    const half2_t s2 = as_half2(__builtin_amdgcn_perm(w, w, 0x000C000Cu));
    const uint4_t u = {as_u32(e0 * s2), as_u32(e1 * s2), as_u32(e2 * s2), as_u32(e3 * s2)};
    return __builtin_bit_cast(half8_t, u);
}

// One GF4 word -> 8 biased exact fp16 values P_i = base_i + q_i in column
// order 0,4,1,5,2,6,3,7 (6 VALU ops, no scale):
//   (64 + q0, 1024 + q4) (8 + q1, 128 + q5) (64 + q2, 1024 + q6) (8 + q3, 128 + q7).
// The level of column i is 4 - q_i = kGf4Bias[slot] - P_slot, where
// kGf4Bias = 4 + base per slot; the word's weight is (4 - q_i) * s / 4.
__device__ __forceinline__ half8_t gf4_word_to_biased(uint32_t w, const Gf4Consts& c) {
    const uint32_t t1 = w >> 4;
    const uint32_t t2 = w >> 10;
    const uint4_t u = {and_xor(t1, c.mask_a, c.magic_a), and_xor(t1, c.mask_b, c.magic_b),
                       and_xor(t2, c.mask_a, c.magic_a), and_xor(t2, c.mask_b, c.magic_b)};
    return __builtin_bit_cast(half8_t, u);
}

// 4 + base of each slot of gf4_word_to_biased.
__device__ __forceinline__ float gf4_bias(int slot) {
    return (slot & 1) ? ((slot & 2) ? 132.0f : 1028.0f) : ((slot & 2) ? 12.0f : 68.0f);
}

// The word's e5m2 scale as fp32 (v_cvt_f32_bf8 of byte 0: OCP E5M2 is the
// high byte of an IEEE binary16, so this is exactly fp16(b << 8)).
__device__ __forceinline__ float gf4_scale_f32(uint32_t w) {
    return __builtin_amdgcn_cvt_f32_bf8((int)w, 0);
}

}  // namespace qw35
