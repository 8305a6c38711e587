// fp32 (or fp16) dequantisation of GF4 / GF2 / q8_0 / Q4_K / Q5_K / Q6_K / F16 tensors,
// optionally gathering rows.
//
// This is the library's bit-exact statement of each format (every weight of
// all three codecs is exact in fp32, so results are compared bit-for-bit with
// the CPU oracle).  With a row list it is the embedding row gather of
// qw35_get_row(s)_{q8_0,q4_k}_f32 (qw35-server/src/metal/qw35_matvec.metal:100-169).
//
//   GF4  (tools/qw35_cook_common.py:79):  w = (4 - (c ^ 4)) * 0.25 * s, s = fp16(b << 8)
//   GF2  (qw35_gf2.metal:19-50):          w = (q * fl(2/3) - 1) * s in fp32 steps, s = fp16(b << 8)
//   q8_0 (qw35_types.metal:24-36):        w = fp32(d) * qs[i]
//   Q4_K (qw35_matvec.metal:2-12):        w = d * sc_j * q - dmin * m_j
//   Q5_K (qw35_matvec.metal:40-62):       the same with q = nibble | (bit j of qh[e % 32]) << 4
//   Q6_K (qw35_matvec.metal:458-542):     w = (d * sc[e/16]) * (q - 32), q = ql nibble | qh 2 bits << 4
//                                         (exact; the reference tile form qw35_dequantize_q6_k,
//                                         :65-98, agrees in value)
#include "qw35_device.h"
#include "qw35_kernels.h"

namespace qw35 {
namespace {

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// One thread per output group of 8 columns; F16_OUT writes fp16 RNE of the
// same values (the prefill image of a quantised weight).
// A gathered row id >= rows yields a row of zeros (no out-of-bounds read).
template <bool F16_OUT>
__global__ __launch_bounds__(256) void dequant_kernel(uint32_t type_id, const uint8_t* __restrict__ w, int rows,
                                                      int k, const uint32_t* __restrict__ row_ids, int n_out_rows,
                                                      void* __restrict__ dst) {
    const int groups = k >> 3;
    const size_t gid = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (size_t)n_out_rows * groups) return;
    const int out_row = (int)(gid / groups);
    const int g = (int)(gid % groups);
    const size_t src_row = row_ids ? (size_t)row_ids[out_row] : (size_t)out_row;
    float v[8];
    if (src_row >= (size_t)rows) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    } else if (type_id == kTypeGF4) {
        const uint32_t word = reinterpret_cast<const uint32_t*>(w)[src_row * groups + g];
        const float s = f16_to_f32((word & 0xFFu) << 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t q = ((word >> (8 + 3 * i)) & 7u) ^ 4u;
            v[i] = (4.0f - (float)q) * 0.25f * s;
        }
    } else if (type_id == kTypeGF2) {
        // 80-byte super-blocks of 256 columns: 16 code words, then their 16 scale bytes
        const int col = 8 * g;
        const uint8_t* blk = w + src_row * (size_t)(k >> 8) * 80 + (size_t)(col >> 8) * 80;
        const int wi = (col & 255) >> 4;
        const uint32_t word = reinterpret_cast<const uint32_t*>(blk)[wi] >> (2 * (col & 15));
        const float s = f16_to_f32((uint32_t)blk[64 + wi] << 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float lev = __fsub_rn(__fmul_rn((float)((word >> (2 * i)) & 3u), 2.0f / 3.0f), 1.0f);
            v[i] = __fmul_rn(lev, s);
        }
    } else if (type_id == kTypeQ8_0) {
        const uint8_t* row = w + src_row * (size_t)(k >> 5) * 34;
        const int col = 8 * g;
        const uint8_t* blk = row + (size_t)(col >> 5) * 34;
        const float d = f16_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = d * (float)(int8_t)blk[2 + (col & 31) + i];
    } else if (type_id == kTypeF16) {
        const uint4_t u = *reinterpret_cast<const uint4_t*>(w + (src_row * (size_t)k + 8 * g) * 2);
        const uint32_t h[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = f16_to_f32(h[i] & 0xFFFFu);
            v[2 * i + 1] = f16_to_f32(h[i] >> 16);
        }
    } else if (type_id == kTypeQ6_K) {
        const uint8_t* row = w + src_row * (size_t)(k >> 8) * 210;
        const int col = 8 * g;
        const uint8_t* blk = row + (size_t)(col >> 8) * 210;
        const int e0 = col & 255;
        const float d = f16_to_f32((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
        const float dsc = d * (float)(int8_t)blk[192 + (e0 >> 4)];  // 8 columns within one sub-block
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + i;
            const int h = e >> 7, gg = (e & 127) >> 5, l = e & 31;
            const uint32_t lo = (blk[64 * h + 32 * (gg & 1) + l] >> (4 * (gg >> 1))) & 15u;
            const uint32_t hi = (blk[128 + 32 * h + l] >> (2 * gg)) & 3u;
            v[i] = dsc * (float)((int)(lo | (hi << 4)) - 32);
        }
    } else {  // Q4_K, Q5_K
        const bool q5 = type_id == kTypeQ5_K;
        const size_t bb = q5 ? 176 : 144;
        const uint8_t* row = w + src_row * (size_t)(k >> 8) * bb;
        const int col = 8 * g;
        const uint8_t* blk = row + (size_t)(col >> 8) * bb;
        const int e = col & 255;
        const int j = e >> 5;
        const uint8_t* sc = blk + 4;
        uint32_t s6, m6;
        if (j < 4) {
            s6 = sc[j] & 63;
            m6 = sc[j + 4] & 63;
        } else {
            s6 = (sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4);
            m6 = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
        }
        const float d = f16_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        const float dmin = f16_to_f32((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
        const float dsc = d * (float)s6;
        const float mm = dmin * (float)m6;
        const uint8_t* qs = blk + (q5 ? 48 : 16) + (j >> 1) * 32 + (e & 31);
        const uint8_t* qh = blk + 16 + (e & 31);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t q = (j & 1) ? (qs[i] >> 4) : (qs[i] & 0x0F);
            if (q5) q |= ((qh[i] >> j) & 1u) << 4;
            v[i] = dsc * (float)q - mm;
        }
    }
    if constexpr (F16_OUT) {
        uint16_t* o = static_cast<uint16_t*>(dst) + (size_t)out_row * k + 8 * g;
        *reinterpret_cast<uint4_t*>(o) =
            uint4_t{as_u32(h2(v[0], v[1])), as_u32(h2(v[2], v[3])), as_u32(h2(v[4], v[5])), as_u32(h2(v[6], v[7]))};
    } else {
        float* o = static_cast<float*>(dst) + (size_t)out_row * k + 8 * g;
        *reinterpret_cast<float4_t*>(o) = float4_t{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<float4_t*>(o + 4) = float4_t{v[4], v[5], v[6], v[7]};
    }
}

}  // namespace

hipError_t launch_dequant(uint32_t type_id, const void* w, int rows, int k, const uint32_t* row_ids,
                          int n_out_rows, void* dst, bool f16_out, hipStream_t stream) {
    const size_t total = (size_t)n_out_rows * (size_t)(k >> 3);
    if (total == 0) return hipSuccess;
    const unsigned grid = (unsigned)((total + 255) / 256);
    if (f16_out)
        hipLaunchKernelGGL((dequant_kernel<true>), dim3(grid), dim3(256), 0, stream, type_id,
                           static_cast<const uint8_t*>(w), rows, k, row_ids, n_out_rows, dst);
    else
        hipLaunchKernelGGL((dequant_kernel<false>), dim3(grid), dim3(256), 0, stream, type_id,
                           static_cast<const uint8_t*>(w), rows, k, row_ids, n_out_rows, dst);
    return hipGetLastError();
}

}  // namespace qw35
