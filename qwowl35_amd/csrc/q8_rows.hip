// q8_0 decode GEMV and fused gate/up/SwiGLU for rows whose length k is a
// multiple of 32 columns but not of 256.  The chunked kernel (kquant_mfma.h)
// needs k % 256 == 0: it works in 256-column chunks and loads each row as
// 16-byte segments, while a q8_0 row of k % 256 != 0 is k/32 x 34 bytes and
// only 2-byte aligned.  The reference decodes any such row
// (qw35_decode_matmul_q8_0{,_residual}_f32, qw35_matvec.metal:630-683, with
// n_blocks = ceil(k / 32), Qw35MetalRuntime+FFN.m:240).
//
// A workgroup of kRowWaves waves owns kRowWaves * RW rows (RW rows per wave)
// and walks K in chunks of 64 blocks (2048 columns):
// * the chunk's activations, times AWQ, are staged once per workgroup in LDS,
//   36 floats per 32-column block (4 of padding, so the lanes' 16-byte reads
//   of 16 consecutive blocks touch 64 distinct banks);
// * lane l takes block l of the chunk in each of its wave's RW rows: the 34
//   bytes come as two dwordx4 loads from the 4-byte boundary at or 2 bytes
//   before the block and two ushort loads of its last four bytes, realigned
//   with v_alignbyte;
// * per 4-column group the lane reads the activations of all batch rows from
//   LDS once and applies them to its RW rows' weights (int8 -> fp32), and
//   y[b] (+)= sum_blocks d * sum_i q_i x_i in fp32, then a wave sum per row.
// No Qwen3.5 projection has such a k; the kernel keeps the fp32 arithmetic of
// the reference's and favours simplicity over the last bytes per second.
#include "qw35_device.h"
#include "qw35_kernels.h"

#include <stdio.h>

namespace qw35 {
namespace {

constexpr int kRowWaves = 8;     // waves per workgroup
constexpr int kChunkBlocks = 64;  // 32-column blocks per K chunk: one per lane
constexpr int kXStride = 36;     // floats per staged block (32 + 4 padding)

typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

// Rows per wave.  Two at batch 4..8 halve the LDS activation reads per weight
// byte; one otherwise (and for the fused gate/up, two matrices per row) keeps
// more workgroups in the grid.  Measured (us, 4096 / 12288 / 24576 x 4160):
// batch 1 8.1 / 18.9 / 31.9 and batch 8 17.6 / 39.1 / 70.4, against 12.4 /
// 20.1 / 33.8 and 26.5 / 58.1 / 91.7 with four rows per wave.
template <int NB, bool SWIGLU>
constexpr int rows_per_wave() {
    return SWIGLU ? 1 : (NB >= 4 ? 2 : 1);
}

template <int NB, bool SWIGLU, bool HAS_AWQ>
__global__ __launch_bounds__(64 * kRowWaves) void q8_gemv_rows(GemvArgs args) {
    constexpr int NM = SWIGLU ? 2 : 1;
    constexpr int RW = rows_per_wave<NB, SWIGLU>();
    extern __shared__ __attribute__((aligned(16))) float xs[];  // [NB][kChunkBlocks * kXStride]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int k = args.k;
    const int n_batch = args.n_batch;
    const int nblk = k >> 5;
    const size_t row_bytes = (size_t)nblk * 34;

    // This wave's rows: their matrices, outputs and segment row counts (a
    // merged launch lists the segments' rows one after another).
    const uint8_t* wrow[NM][RW];
    float* yrow[RW];
    int ystride[RW];
    bool live[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        int row = ((int)blockIdx.x * kRowWaves + wave) * RW + r;
        const void* wm = args.w;
        float* yout = args.y;
        int rows = args.rows;
        if (args.n_seg > 1) {
            int s = 0;
            while (s < args.n_seg - 1 && row >= args.seg_rows[s]) row -= args.seg_rows[s++];
            wm = args.seg_w[s];
            yout = args.seg_y[s];
            rows = args.seg_rows[s];
        }
        live[r] = row < rows;
        const int rr = live[r] ? row : 0;  // rows past the matrix re-read its first row (never stored)
        wrow[0][r] = static_cast<const uint8_t*>(wm) + (size_t)rr * row_bytes;
        if constexpr (SWIGLU) wrow[NM - 1][r] = static_cast<const uint8_t*>(args.w_up) + (size_t)rr * row_bytes;
        yrow[r] = yout + rr;
        ystride[r] = rows;
    }

    float acc[NM][RW][NB];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[m][r][b] = 0.0f;

    for (int c0 = 0; c0 < nblk; c0 += kChunkBlocks) {
        const int cb = min(kChunkBlocks, nblk - c0);
        __syncthreads();  // the previous chunk's activations are no longer read
        // Stage this chunk's activations (times AWQ): NB x cb blocks x 8 groups of 4.
        for (int it = threadIdx.x; it < NB * cb * 8; it += 64 * kRowWaves) {
            const int b = it / (cb * 8);
            const int rem = it - b * cb * 8;
            const int j = rem >> 3;
            const int g = rem & 7;
            const int col = (c0 + j) * 32 + 4 * g;
            const int bb = b < n_batch ? b : 0;  // batch rows past n_batch re-read row 0 (never stored)
            float4_t v = *reinterpret_cast<const float4_t*>(args.x + (size_t)bb * k + col);
            if constexpr (HAS_AWQ) v *= *reinterpret_cast<const float4_t*>(args.awq + col);
            *reinterpret_cast<float4_t*>(xs + (size_t)b * kChunkBlocks * kXStride + j * kXStride + 4 * g) = v;
        }
        __syncthreads();
        if (lane >= cb) continue;
        const size_t boff = (size_t)(c0 + lane) * 34;
        // The lane's block of each row: d and the 32 codes as 8 dwords.
        float d[NM][RW];
        uint32_t q[NM][RW][8];
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const uint8_t* bp = wrow[m][r] + boff;
                const uint32_t off = (uint32_t)((uintptr_t)bp & 3u);  // 0 or 2
                const uint32_t* a = reinterpret_cast<const uint32_t*>(bp - off);
                const u32x4_a4 v0 = *reinterpret_cast<const u32x4_a4*>(a);
                const u32x4_a4 v1 = *reinterpret_cast<const u32x4_a4*>(a + 4);
                // dword 8 of the window from the block's last four bytes (two ushort
                // loads: nothing past the block is read, whatever its alignment)
                const uint32_t t30 = *reinterpret_cast<const uint16_t*>(bp + 30);
                const uint32_t t32 = *reinterpret_cast<const uint16_t*>(bp + 32);
                const uint32_t v2 = off ? (t30 | t32 << 16) : t32;
                const uint32_t w[9] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, v2};
                d[m][r] = (float)__builtin_bit_cast(_Float16,
                                                    (uint16_t)__builtin_amdgcn_alignbyte(w[1], w[0], off));
                // codes from byte off + 2: dword t is w[t + 1] (off = 2) or straddles
                // w[t] and w[t + 1] (off = 0; v_alignbyte takes its shift mod 4)
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    q[m][r][t] = off ? w[t + 1] : __builtin_amdgcn_alignbyte(w[t + 1], w[t], 2);
            }
        float part[NM][RW][NB];
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int b = 0; b < NB; ++b) part[m][r][b] = 0.0f;
#pragma unroll
        for (int g = 0; g < 8; ++g) {  // columns 32 j + 4 g .. + 3
            float4_t x4[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b)
                x4[b] = *reinterpret_cast<const float4_t*>(xs + (size_t)b * kChunkBlocks * kXStride +
                                                           lane * kXStride + 4 * g);
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    // int8 -> fp32 (an int8_t cast: __builtin_amdgcn_sbfe returns unsigned,
                    // so its (float) would convert the sign-extended byte as unsigned)
                    float w4[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) w4[i] = (float)(int8_t)(q[m][r][g] >> (8 * i));
#pragma unroll
                    for (int b = 0; b < NB; ++b)
#pragma unroll
                        for (int i = 0; i < 4; ++i) part[m][r][b] = __builtin_fmaf(w4[i], x4[b][i], part[m][r][b]);
                }
        }
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int b = 0; b < NB; ++b) acc[m][r][b] = __builtin_fmaf(d[m][r], part[m][r][b], acc[m][r][b]);
    }

#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) acc[m][r][b] += __shfl_xor(acc[m][r][b], o);
            }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            if (!live[r]) continue;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b >= n_batch) break;
                float* yp = yrow[r] + (size_t)b * ystride[r];
                float v = SWIGLU ? silu(acc[0][r][b]) * acc[NM - 1][r][b] : acc[0][r][b];
                if (args.residual) v += *yp;
                *yp = v;
            }
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
    constexpr int rows_per_group = kRowWaves * rows_per_wave<NB, SWIGLU>();
    const int grid = (total + rows_per_group - 1) / rows_per_group;
    const size_t lds = (size_t)NB * kChunkBlocks * kXStride * sizeof(float);
    if (a.info) {
        snprintf(a.info->name, sizeof a.info->name, "q8_gemv_rows<%d, %s, %s>", NB, SWIGLU ? "true" : "false",
                 a.awq ? "true" : "false");
        a.info->grid = (unsigned)grid;
        a.info->block = 64u * kRowWaves;
        a.info->lds = (unsigned)lds;
        a.info->splits = 1;
        a.info->ws_bytes = 0;
        return hipSuccess;
    }
    if (a.awq)
        hipLaunchKernelGGL((q8_gemv_rows<NB, SWIGLU, true>), dim3(grid), dim3(64 * kRowWaves), lds, stream, a);
    else
        hipLaunchKernelGGL((q8_gemv_rows<NB, SWIGLU, false>), dim3(grid), dim3(64 * kRowWaves), lds, stream, a);
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
