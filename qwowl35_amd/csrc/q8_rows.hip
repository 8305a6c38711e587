// q8_0 decode GEMV and fused gate/up/SwiGLU for rows whose length k is a
// multiple of 32 columns but not of 256.  The chunked kernel (kquant_mfma.h)
// needs k % 256 == 0: it works in 256-column chunks and loads each row as
// 16-byte segments, while a q8_0 row of k % 256 != 0 is k/32 x 34 bytes and
// only 2-byte aligned.  The reference decodes any such row
// (qw35_decode_matmul_q8_0{,_residual}_f32, qw35_matvec.metal:630-683, with
// n_blocks = ceil(k / 32), Qw35MetalRuntime+FFN.m:240).
//
// One wave per row; lane l takes blocks l, l + 64, ...: d and the 32 int8
// codes are read as 2-byte words (naturally aligned for any row), and
// y[b] (+)= sum_j d_j * sum_i q_ji * awq_i * x[b]_i in fp32, then a wave sum.
// Bandwidth is secondary here: no Qwen3.5 projection has such a k.
#include "qw35_device.h"
#include "qw35_kernels.h"

#include <stdio.h>

namespace qw35 {
namespace {

constexpr int kRowWaves = 4;  // rows (one per wave) per workgroup

template <int NB, bool SWIGLU, bool HAS_AWQ>
__global__ __launch_bounds__(64 * kRowWaves) void q8_gemv_rows(GemvArgs args) {
    constexpr int NM = SWIGLU ? 2 : 1;
    const int lane = threadIdx.x & 63;
    int row = (int)blockIdx.x * kRowWaves + (int)(threadIdx.x >> 6);
    const void* wm = args.w;
    float* yout = args.y;
    int rows = args.rows;
    if (args.n_seg > 1) {  // merged launch: rows of the segments one after another
        int s = 0;
        while (s < args.n_seg - 1 && row >= args.seg_rows[s]) row -= args.seg_rows[s++];
        wm = args.seg_w[s];
        yout = args.seg_y[s];
        rows = args.seg_rows[s];
    }
    if (row >= rows) return;  // the whole wave
    const int k = args.k;
    const int n_batch = args.n_batch;
    const int nblk = k >> 5;
    const size_t row_bytes = (size_t)nblk * 34;
    float acc[NM][NB];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[m][b] = 0.0f;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const uint8_t* wr = static_cast<const uint8_t*>(m == 0 ? wm : args.w_up) + (size_t)row * row_bytes;
        for (int j = lane; j < nblk; j += 64) {
            const uint16_t* bp = reinterpret_cast<const uint16_t*>(wr + (size_t)j * 34);
            const float d = (float)__builtin_bit_cast(_Float16, bp[0]);
            float part[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) part[b] = 0.0f;
#pragma unroll
            for (int g = 0; g < 8; ++g) {  // columns 32j + 4g .. +3
                const uint32_t q4 = (uint32_t)bp[1 + 2 * g] | ((uint32_t)bp[2 + 2 * g] << 16);
                float w4[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) w4[r] = (float)(int8_t)(q4 >> (8 * r));
                const int col = 32 * j + 4 * g;
                if constexpr (HAS_AWQ) {
                    const float4_t s4 = *reinterpret_cast<const float4_t*>(args.awq + col);
#pragma unroll
                    for (int r = 0; r < 4; ++r) w4[r] *= s4[r];
                }
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const int bb = b < n_batch ? b : 0;  // rows past the batch re-read row 0 (never stored)
                    const float4_t x4 = *reinterpret_cast<const float4_t*>(args.x + (size_t)bb * k + col);
#pragma unroll
                    for (int r = 0; r < 4; ++r) part[b] = __builtin_fmaf(w4[r], x4[r], part[b]);
                }
            }
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[m][b] = __builtin_fmaf(d, part[b], acc[m][b]);
        }
    }
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) acc[m][b] += __shfl_xor(acc[m][b], o);
        }
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b >= n_batch) break;
            float* yp = yout + (size_t)b * rows + row;
            float v = SWIGLU ? silu(acc[0][b]) * acc[NM - 1][b] : acc[0][b];
            if (args.residual) v += *yp;
            *yp = v;
        }
    }
}

template <int NB, bool SWIGLU>
hipError_t launch_rows_nb(const GemvArgs& a, hipStream_t stream) {
    int total = a.rows;
    if (a.n_seg > 1) {
        total = 0;
        for (int s = 0; s < a.n_seg; ++s) total += a.seg_rows[s];
    }
    const int grid = (total + kRowWaves - 1) / kRowWaves;
    if (a.info) {
        snprintf(a.info->name, sizeof a.info->name, "q8_gemv_rows<%d, %s, %s>", NB, SWIGLU ? "true" : "false",
                 a.awq ? "true" : "false");
        a.info->grid = (unsigned)grid;
        a.info->block = 64u * kRowWaves;
        a.info->lds = 0;
        a.info->splits = 1;
        a.info->ws_bytes = 0;
        return hipSuccess;
    }
    if (a.awq)
        hipLaunchKernelGGL((q8_gemv_rows<NB, SWIGLU, true>), dim3(grid), dim3(64 * kRowWaves), 0, stream, a);
    else
        hipLaunchKernelGGL((q8_gemv_rows<NB, SWIGLU, false>), dim3(grid), dim3(64 * kRowWaves), 0, stream, a);
    return hipGetLastError();
}

template <bool SWIGLU>
hipError_t launch_rows(const GemvArgs& a, hipStream_t stream) {
    if (a.n_batch <= 1) return launch_rows_nb<1, SWIGLU>(a, stream);
    if (a.n_batch == 2) return launch_rows_nb<2, SWIGLU>(a, stream);
    if (a.n_batch <= 4) return launch_rows_nb<4, SWIGLU>(a, stream);
    return launch_rows_nb<8, SWIGLU>(a, stream);
}

}  // namespace

hipError_t launch_q8_0_gemv_rows(const GemvArgs& a, hipStream_t stream) {
    if (a.am_token || (a.k & 31) != 0) return hipErrorInvalidValue;  // no greedy-head epilogue here
    return a.w_up ? launch_rows<true>(a, stream) : launch_rows<false>(a, stream);
}

}  // namespace qw35
