// Weight producers: fp32 matrix -> GF4 / GF2 / q8_0 / Q4_K / Q5_K / Q6_K / F16 tensor bytes, on the GPU.
//
// GF4 is the reference packer pack_gf4_prepared(rows, scale_search=False)
// (tools/qw35_cook_common.py:83-119), including the optional AWQ column
// multiply that pack_ffn_gf4 applies before packing (:182-199, the multiply
// at :198).  Every step is an IEEE fp32 / binary16 operation with the same
// rounding as the numpy statement, so the words are bit-identical:
//   gmax  = first element of the 8-group with the largest |x|, with its sign
//   b     = (bits(fp16_rne(gmax)) + 0x80) >> 8          (e5m2 byte, :48-51)
//   s     = fp16(b << 8)                                (:54-56)
//   q_raw = clip(rint(fl(x / s) * -4 + 4), 0, 7), 0 where s == 0   (:67-80)
//   word  = b | sum_i (q_raw_i ^ 4) << (8 + 3 i)        (:113-118)
// q8_0, Q4_K, Q5_K and Q6_K have no encoder in the reference (it reads them through
// the external gguf-py); these are this library's own min/max encoders, the GPU
// statement of the ones the tests use, producing valid GGUF blocks.
//
// Inputs must be finite: NaN ordering in numpy's argmax and its float->int
// casts are platform behaviour, not part of the format.
#include "qw35_device.h"
#include "qw35_kernels.h"

namespace qw35 {
namespace {

__device__ __forceinline__ uint32_t f32_to_f16_bits(float v) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// Grid-stride loops keep the grid at a fixed size for any tensor.
constexpr int kEncodeThreads = 256;
constexpr int kEncodeBlocks = 2048;

// One thread per GF4 word (8 consecutive columns of a row).
__global__ __launch_bounds__(kEncodeThreads) void gf4_pack_kernel(const float* __restrict__ src,
                                                                  const float* __restrict__ col_scale,
                                                                  uint32_t* __restrict__ dst, uint64_t n_words,
                                                                  uint32_t words_per_row) {
    for (uint64_t i = (uint64_t)blockIdx.x * kEncodeThreads + threadIdx.x; i < n_words;
         i += (uint64_t)gridDim.x * kEncodeThreads) {
        const float4_t lo = *reinterpret_cast<const float4_t*>(src + 8 * i);
        const float4_t hi = *reinterpret_cast<const float4_t*>(src + 8 * i + 4);
        float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        if (col_scale) {
            const uint32_t c0 = 8u * (uint32_t)(i % words_per_row);
            const float4_t s0 = *reinterpret_cast<const float4_t*>(col_scale + c0);
            const float4_t s1 = *reinterpret_cast<const float4_t*>(col_scale + c0 + 4);
            const float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = __fmul_rn(v[j], s[j]);
        }
        int best = 0;
        float best_abs = fabsf(v[0]);
#pragma unroll
        for (int j = 1; j < 8; ++j) {
            if (fabsf(v[j]) > best_abs) {  // strict: the first maximum wins
                best_abs = fabsf(v[j]);
                best = j;
            }
        }
        float gmax = v[0];
#pragma unroll
        for (int j = 1; j < 8; ++j)
            if (j == best) gmax = v[j];
        const uint32_t b = ((f32_to_f16_bits(gmax) + 0x80u) >> 8) & 0xFFu;
        const float s = f16_bits_to_f32(b << 8);
        uint32_t word = b;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float ratio = (s != 0.0f) ? __fdiv_rn(v[j], s) : 0.0f;
            const float t = __fadd_rn(__fmul_rn(ratio, -4.0f), 4.0f);
            const float q = fminf(fmaxf(rintf(t), 0.0f), 7.0f);
            word |= (((uint32_t)q) ^ 4u) << (8 + 3 * j);
        }
        dst[i] = word;
    }
}

// One thread per q8_0 block: d = max|x| / 127, q = round_half_away(x * (1/d)).
// One thread per GF2 super-block (256 columns = 16 groups of 16; this library's
// encoder, the statement of oracle gf2_quantize):
//   b = e5m2(max |x|) (fp16 RNE, low byte rounded half-up), s = fp16(b << 8)
//   t = x / s (0 where s == 0), q = clip(rint(t * 1.5 + 1.5), 0, 3)
// written as the reference's super-block: 16 code words (code i of word w in
// bits 2i, 2i+1 for column 16w + i) then the 16 scale bytes
// (qw35-server/src/metal/qw35_gf2.metal:1-17).
__global__ __launch_bounds__(kEncodeThreads) void gf2_pack_kernel(const float* __restrict__ src,
                                                                  const float* __restrict__ col_scale,
                                                                  uint8_t* __restrict__ dst, uint64_t n_blocks,
                                                                  uint32_t blocks_per_row) {
    for (uint64_t i = (uint64_t)blockIdx.x * kEncodeThreads + threadIdx.x; i < n_blocks;
         i += (uint64_t)gridDim.x * kEncodeThreads) {
        const float* x = src + 256 * i;
        const float* cs = col_scale ? col_scale + 256u * (uint32_t)(i % blocks_per_row) : nullptr;
        uint32_t words[16];
        uint32_t sb[4] = {0, 0, 0, 0};
        for (int w = 0; w < 16; ++w) {
            float v[16];
            float amax = 0.0f;
            for (int l = 0; l < 16; ++l) {
                v[l] = cs ? __fmul_rn(x[16 * w + l], cs[16 * w + l]) : x[16 * w + l];
                amax = fmaxf(amax, fabsf(v[l]));
            }
            const uint32_t b = ((f32_to_f16_bits(amax) + 0x80u) >> 8) & 0xFFu;
            const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)(b << 8));
            uint32_t word = 0;
            for (int l = 0; l < 16; ++l) {
                const float t = s != 0.0f ? __fdiv_rn(v[l], s) : 0.0f;
                const float q = fminf(fmaxf(rintf(__fadd_rn(__fmul_rn(t, 1.5f), 1.5f)), 0.0f), 3.0f);
                word |= (uint32_t)q << (2 * l);
            }
            words[w] = word;
            sb[w >> 2] |= b << (8 * (w & 3));
        }
        uint4_t* o = reinterpret_cast<uint4_t*>(dst + 80 * i);  // 80-byte blocks: 16-byte aligned
        for (int q = 0; q < 4; ++q) o[q] = uint4_t{words[4 * q], words[4 * q + 1], words[4 * q + 2], words[4 * q + 3]};
        o[4] = uint4_t{sb[0], sb[1], sb[2], sb[3]};
    }
}

__global__ __launch_bounds__(kEncodeThreads) void q8_0_quantize_kernel(const float* __restrict__ src,
                                                                       const float* __restrict__ col_scale,
                                                                       uint8_t* __restrict__ dst, uint64_t n_blocks,
                                                                       uint32_t blocks_per_row) {
    for (uint64_t i = (uint64_t)blockIdx.x * kEncodeThreads + threadIdx.x; i < n_blocks;
         i += (uint64_t)gridDim.x * kEncodeThreads) {
        float v[32];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4_t t = *reinterpret_cast<const float4_t*>(src + 32 * i + 4 * j);
            v[4 * j] = t.x;
            v[4 * j + 1] = t.y;
            v[4 * j + 2] = t.z;
            v[4 * j + 3] = t.w;
        }
        if (col_scale) {
            const float* cs = col_scale + 32u * (uint32_t)(i % blocks_per_row);
#pragma unroll
            for (int j = 0; j < 32; ++j) v[j] = __fmul_rn(v[j], cs[j]);
        }
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
        const float d = __fdiv_rn(amax, 127.0f);
        const float inv = (d != 0.0f) ? __fdiv_rn(1.0f, d) : 0.0f;
        uint8_t* blk = dst + 34 * i;  // 34-byte blocks: 2-byte aligned
        uint16_t* h = reinterpret_cast<uint16_t*>(blk);
        h[0] = (uint16_t)f32_to_f16_bits(d);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            int q2[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const float sc = __fmul_rn(v[2 * j + u], inv);
                float q = truncf(__fadd_rn(sc, copysignf(0.5f, sc)));
                q = fminf(fmaxf(q, -127.0f), 127.0f);
                q2[u] = (int)q;
            }
            h[1 + j] = (uint16_t)((uint32_t)(q2[0] & 0xFF) | ((uint32_t)(q2[1] & 0xFF) << 8));
        }
    }
}

// One thread per Q4_K (Q5_K) super-block (256 columns, 8 sub-blocks of 32),
// with L = 15 (31) code levels:
//   lo_j = min(min(x), 0), hi_j = max(x), scale_j = (hi_j - lo_j) / L, min_j = -lo_j
//   d = fp16(max_j scale_j / 63), dmin = fp16(max_j min_j / 63)
//   sc_j = clip(rint(scale_j / d), 0, 63), m_j = clip(rint(min_j / dmin), 0, 63)
//   q = clip(rint((x + dmin*m_j) / (d*sc_j)), 0, L)
// with the 12-byte 6-bit scale packing of get_scale_min_k4
// (qw35-server/src/metal/qw35_matvec.metal:2-12) and the nibble layout
// qs[32c + l] = q[64c + l] | q[64c + 32 + l] << 4 (low nibbles only for Q5_K,
// whose qs starts at byte 48; bit 4 of q for element 32j + l is bit j of qh[l],
// qh at byte 16; qw35_types.metal:9-15).
template <bool Q5>
__global__ __launch_bounds__(kEncodeThreads) void k_quantize_kernel(const float* __restrict__ src,
                                                                    const float* __restrict__ col_scale,
                                                                    uint8_t* __restrict__ dst, uint64_t n_blocks,
                                                                    uint32_t blocks_per_row) {
    constexpr float kLevels = Q5 ? 31.0f : 15.0f;
    constexpr int kBlockBytes = Q5 ? 176 : 144;
    constexpr int kQs = Q5 ? 48 : 16;
    for (uint64_t i = (uint64_t)blockIdx.x * kEncodeThreads + threadIdx.x; i < n_blocks;
         i += (uint64_t)gridDim.x * kEncodeThreads) {
        const float* x = src + 256 * i;
        const float* cs = col_scale ? col_scale + 256u * (uint32_t)(i % blocks_per_row) : nullptr;
        float scale[8], mins[8];
        for (int j = 0; j < 8; ++j) {
            float lo = INFINITY, hi = -INFINITY;
            for (int l = 0; l < 32; ++l) {
                const float v = cs ? __fmul_rn(x[32 * j + l], cs[32 * j + l]) : x[32 * j + l];
                lo = fminf(lo, v);
                hi = fmaxf(hi, v);
            }
            lo = fminf(lo, 0.0f);
            scale[j] = __fdiv_rn(__fsub_rn(hi, lo), kLevels);
            mins[j] = -lo;
        }
        float smax = scale[0], mmax = mins[0];
        for (int j = 1; j < 8; ++j) {
            smax = fmaxf(smax, scale[j]);
            mmax = fmaxf(mmax, mins[j]);
        }
        const uint32_t d_bits = f32_to_f16_bits(__fdiv_rn(smax, 63.0f));
        const uint32_t dmin_bits = f32_to_f16_bits(__fdiv_rn(mmax, 63.0f));
        const float df = f16_bits_to_f32(d_bits);
        const float dminf = f16_bits_to_f32(dmin_bits);
        uint32_t sc[8], mq[8];
        float step[8], offs[8];
        for (int j = 0; j < 8; ++j) {
            const float a = (df != 0.0f) ? rintf(__fdiv_rn(scale[j], df)) : 0.0f;
            const float m = (dminf != 0.0f) ? rintf(__fdiv_rn(mins[j], dminf)) : 0.0f;
            sc[j] = (uint32_t)fminf(fmaxf(a, 0.0f), 63.0f);
            mq[j] = (uint32_t)fminf(fmaxf(m, 0.0f), 63.0f);
            step[j] = __fmul_rn(df, (float)sc[j]);
            offs[j] = __fmul_rn(dminf, (float)mq[j]);
        }
        uint8_t* blk = dst + kBlockBytes * i;  // 144- or 176-byte blocks: 16-byte aligned
        uint32_t head[4];
        head[0] = d_bits | (dmin_bits << 16);
        uint8_t scales[12];
        for (int j = 0; j < 4; ++j) {
            scales[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            scales[j + 4] = (uint8_t)((mq[j] & 63) | ((mq[j + 4] >> 4) << 6));
            scales[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mq[j + 4] & 0xF) << 4));
        }
        for (int w = 0; w < 3; ++w)
            head[1 + w] = (uint32_t)scales[4 * w] | ((uint32_t)scales[4 * w + 1] << 8) |
                          ((uint32_t)scales[4 * w + 2] << 16) | ((uint32_t)scales[4 * w + 3] << 24);
        *reinterpret_cast<uint4_t*>(blk) = uint4_t{head[0], head[1], head[2], head[3]};
        uint32_t qh[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // Q5_K: 32 bytes
        for (int c = 0; c < 4; ++c) {
            for (int l4 = 0; l4 < 32; l4 += 16) {
                uint32_t packed[4] = {0, 0, 0, 0};
                for (int l = 0; l < 16; ++l) {
                    uint32_t nib[2];
                    for (int h = 0; h < 2; ++h) {
                        const int j = 2 * c + h;
                        const int e = 32 * j + l4 + l;
                        const float v = cs ? __fmul_rn(x[e], cs[e]) : x[e];
                        const float qf = (step[j] != 0.0f) ? __fdiv_rn(__fadd_rn(v, offs[j]), step[j]) : 0.0f;
                        const uint32_t q = (uint32_t)fminf(fmaxf(rintf(qf), 0.0f), kLevels);
                        nib[h] = q & 15u;
                        if (Q5) qh[(l4 + l) >> 2] |= ((q >> 4) << j) << (8 * ((l4 + l) & 3));
                    }
                    packed[l >> 2] |= (nib[0] | (nib[1] << 4)) << (8 * (l & 3));
                }
                *reinterpret_cast<uint4_t*>(blk + kQs + 32 * c + l4) =
                    uint4_t{packed[0], packed[1], packed[2], packed[3]};
            }
        }
        if (Q5) {
            *reinterpret_cast<uint4_t*>(blk + 16) = uint4_t{qh[0], qh[1], qh[2], qh[3]};
            *reinterpret_cast<uint4_t*>(blk + 32) = uint4_t{qh[4], qh[5], qh[6], qh[7]};
        }
    }
}

// One thread per Q6_K super-block (256 columns, 16 sub-blocks of 16), the
// statement of oracle q6_k_quantize:
//   sub_s = max|x| / 31, d = fp16(max_s sub_s / 127), sc_s = clip(rint(sub_s / d), 0, 127)
//   q = clip(rint(x / (d * sc_s)), -32, 31) + 32
// stored as ggml lays Q6_K out (qw35_types.metal:17-22): element
// 128h + 32g + l has its low nibble in ql[64h + 32(g&1) + l] (high nibble for
// g >= 2) and its top two bits at bit 2g of qh[32h + l].  Super-blocks are
// 210 bytes (2-byte aligned), so the bytes are stored one at a time.
__global__ __launch_bounds__(kEncodeThreads) void q6_k_quantize_kernel(const float* __restrict__ src,
                                                                       const float* __restrict__ col_scale,
                                                                       uint8_t* __restrict__ dst, uint64_t n_blocks,
                                                                       uint32_t blocks_per_row) {
    for (uint64_t i = (uint64_t)blockIdx.x * kEncodeThreads + threadIdx.x; i < n_blocks;
         i += (uint64_t)gridDim.x * kEncodeThreads) {
        const float* x = src + 256 * i;
        const float* cs = col_scale ? col_scale + 256u * (uint32_t)(i % blocks_per_row) : nullptr;
        auto val = [&](int e) { return cs ? __fmul_rn(x[e], cs[e]) : x[e]; };
        float sub[16];
        float smax = 0.0f;
#pragma unroll
        for (int sb = 0; sb < 16; ++sb) {
            float amax = 0.0f;
            for (int l = 0; l < 16; ++l) amax = fmaxf(amax, fabsf(val(16 * sb + l)));
            sub[sb] = __fdiv_rn(amax, 31.0f);
            smax = fmaxf(smax, sub[sb]);
        }
        const uint32_t d_bits = f32_to_f16_bits(__fdiv_rn(smax, 127.0f));
        const float df = f16_bits_to_f32(d_bits);
        float step[16];
        uint8_t* blk = dst + 210 * i;
#pragma unroll
        for (int sb = 0; sb < 16; ++sb) {
            const float a = (df != 0.0f) ? rintf(__fdiv_rn(sub[sb], df)) : 0.0f;
            const float scq = fminf(fmaxf(a, 0.0f), 127.0f);
            step[sb] = __fmul_rn(df, scq);
            blk[192 + sb] = (uint8_t)(int)scq;
        }
        auto code = [&](int e) {
            const float st = step[e >> 4];
            const float qf = (st != 0.0f) ? rintf(__fdiv_rn(val(e), st)) : 0.0f;
            return (uint32_t)(int)(fminf(fmaxf(qf, -32.0f), 31.0f) + 32.0f);
        };
#pragma unroll
        for (int j = 0; j < 128; ++j) {
            const int h = j >> 6, gp = (j >> 5) & 1, l = j & 31;
            const int e = 128 * h + 32 * gp + l;
            blk[j] = (uint8_t)((code(e) & 15u) | ((code(e + 64) & 15u) << 4));
        }
#pragma unroll
        for (int j = 0; j < 64; ++j) {
            const int h = j >> 5, l = j & 31;
            uint32_t b = 0;
#pragma unroll
            for (int g = 0; g < 4; ++g) b |= (code(128 * h + 32 * g + l) >> 4) << (2 * g);
            blk[128 + j] = (uint8_t)b;
        }
        blk[208] = (uint8_t)(d_bits & 0xFFu);
        blk[209] = (uint8_t)(d_bits >> 8);
    }
}

// F16 (GGUF type 1): fp16 round-to-nearest-even of (col_scale *) x, 8 per thread.
__global__ __launch_bounds__(kEncodeThreads) void f16_quantize_kernel(const float* __restrict__ src,
                                                                      const float* __restrict__ col_scale,
                                                                      uint16_t* __restrict__ dst, uint64_t n_groups,
                                                                      uint32_t groups_per_row) {
    for (uint64_t i = (uint64_t)blockIdx.x * kEncodeThreads + threadIdx.x; i < n_groups;
         i += (uint64_t)gridDim.x * kEncodeThreads) {
        float v[8];
        const float4_t a = *reinterpret_cast<const float4_t*>(src + 8 * i);
        const float4_t b = *reinterpret_cast<const float4_t*>(src + 8 * i + 4);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v[q] = a[q];
            v[4 + q] = b[q];
        }
        if (col_scale) {
            const float* cs = col_scale + 8u * (uint32_t)(i % groups_per_row);
#pragma unroll
            for (int q = 0; q < 8; ++q) v[q] = __fmul_rn(v[q], cs[q]);
        }
        *reinterpret_cast<uint4_t*>(dst + 8 * i) =
            uint4_t{as_u32(h2(v[0], v[1])), as_u32(h2(v[2], v[3])), as_u32(h2(v[4], v[5])), as_u32(h2(v[6], v[7]))};
    }
}

unsigned grid_for(uint64_t n) {
    const uint64_t g = (n + kEncodeThreads - 1) / kEncodeThreads;
    return (unsigned)(g < (uint64_t)kEncodeBlocks ? g : (uint64_t)kEncodeBlocks);
}

}  // namespace

hipError_t launch_quantize(uint32_t type_id, const float* src, int rows, int k, const float* col_scale, void* dst,
                           hipStream_t stream) {
    const uint64_t r = (uint64_t)rows;
    switch (type_id) {
        case kTypeGF4: {
            const uint64_t n = r * (uint64_t)(k / 8);
            hipLaunchKernelGGL(gf4_pack_kernel, dim3(grid_for(n)), dim3(kEncodeThreads), 0, stream, src, col_scale,
                               static_cast<uint32_t*>(dst), n, (uint32_t)(k / 8));
            break;
        }
        case kTypeQ8_0: {
            const uint64_t n = r * (uint64_t)(k / 32);
            hipLaunchKernelGGL(q8_0_quantize_kernel, dim3(grid_for(n)), dim3(kEncodeThreads), 0, stream, src,
                               col_scale, static_cast<uint8_t*>(dst), n, (uint32_t)(k / 32));
            break;
        }
        case kTypeF16: {
            const uint64_t n = r * (uint64_t)(k / 8);
            hipLaunchKernelGGL(f16_quantize_kernel, dim3(grid_for(n)), dim3(kEncodeThreads), 0, stream, src,
                               col_scale, static_cast<uint16_t*>(dst), n, (uint32_t)(k / 8));
            break;
        }
        case kTypeQ6_K: {
            const uint64_t n = r * (uint64_t)(k / 256);
            hipLaunchKernelGGL(q6_k_quantize_kernel, dim3(grid_for(n)), dim3(kEncodeThreads), 0, stream, src,
                               col_scale, static_cast<uint8_t*>(dst), n, (uint32_t)(k / 256));
            break;
        }
        case kTypeGF2: {
            const uint64_t n = r * (uint64_t)(k / 256);
            hipLaunchKernelGGL(gf2_pack_kernel, dim3(grid_for(n)), dim3(kEncodeThreads), 0, stream, src, col_scale,
                               static_cast<uint8_t*>(dst), n, (uint32_t)(k / 256));
            break;
        }
        case kTypeQ5_K: {
            const uint64_t n = r * (uint64_t)(k / 256);
            hipLaunchKernelGGL(k_quantize_kernel<true>, dim3(grid_for(n)), dim3(kEncodeThreads), 0, stream, src,
                               col_scale, static_cast<uint8_t*>(dst), n, (uint32_t)(k / 256));
            break;
        }
        default: {
            const uint64_t n = r * (uint64_t)(k / 256);
            hipLaunchKernelGGL(k_quantize_kernel<false>, dim3(grid_for(n)), dim3(kEncodeThreads), 0, stream, src,
                               col_scale, static_cast<uint8_t*>(dst), n, (uint32_t)(k / 256));
            break;
        }
    }
    return hipGetLastError();
}

}  // namespace qw35

// Streaming-read probe: the measured HBM read ceiling the GEMVs are compared
// with.  Every 16-byte word of `buf` is loaded once (non-temporal, four loads in
// flight per thread) and folded into one XOR per workgroup, written to
// sink[blockIdx.x] so that no load can be elided.
namespace qw35 {
namespace {

constexpr int kReadThreads = 512;

__global__ __launch_bounds__(kReadThreads) void stream_read_kernel(const uint4_t* __restrict__ buf, uint64_t words,
                                                                   uint32_t* __restrict__ sink) {
    uint32_t acc = 0;
    const uint64_t stride = (uint64_t)gridDim.x * kReadThreads;
    uint64_t i = (uint64_t)blockIdx.x * kReadThreads + threadIdx.x;
    for (; i + 3 * stride < words; i += 4 * stride) {
        const uint4_t a = load_stream16(buf + i);
        const uint4_t b = load_stream16(buf + i + stride);
        const uint4_t c = load_stream16(buf + i + 2 * stride);
        const uint4_t d = load_stream16(buf + i + 3 * stride);
        acc ^= (a.x ^ a.y ^ a.z ^ a.w) ^ (b.x ^ b.y ^ b.z ^ b.w) ^ (c.x ^ c.y ^ c.z ^ c.w) ^ (d.x ^ d.y ^ d.z ^ d.w);
    }
    for (; i < words; i += stride) {
        const uint4_t a = load_stream16(buf + i);
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    __shared__ uint32_t red[kReadThreads / 64];
    for (int o = 1; o < 64; o <<= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t v = 0;
        for (int w = 0; w < kReadThreads / 64; ++w) v ^= red[w];
        sink[blockIdx.x] = v;
    }
}

}  // namespace

// About 768 words (12 KiB) per workgroup, at most 16384 workgroups: the fastest
// of the launch shapes measured on MI355X for 25 MB (5.1 us) and 1 GiB (6.9 TB/s).
unsigned stream_read_blocks(uint64_t bytes) {
    uint64_t blocks = bytes / 16 / 768;
    if (blocks > 16384) blocks = 16384;
    return blocks ? (unsigned)blocks : 1u;
}

hipError_t launch_stream_read(const void* buf, uint64_t bytes, uint32_t* sink, hipStream_t stream) {
    hipLaunchKernelGGL(stream_read_kernel, dim3(stream_read_blocks(bytes)), dim3(kReadThreads), 0, stream,
                       static_cast<const uint4_t*>(buf), bytes / 16, sink);
    return hipGetLastError();
}

}  // namespace qw35
