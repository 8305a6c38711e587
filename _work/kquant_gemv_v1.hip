// q8_0 and Q4_K decode GEMVs for gfx950: y[b][r] (+)= sum_k W[r][k] * a[k] * x[b][k].
//
// Reference kernels replaced:
//   qw35_decode_matmul_q8_0{,_residual}_f32      (qw35-server/src/metal/qw35_matvec.metal:630-683)
//   qw35_decode_matmul_q4_k_2row{,_residual}_f32 (qw35-server/src/metal/qw35_matvec.metal:171-353)
//
// Both kernels accumulate in fp32 from fp32 activations (a*x staged once per
// workgroup in LDS); weights are decoded to exact small integers in registers
// and their block scales are applied once per 32-element block.
//
// q8_0: 34-byte blocks (fp16 d, 32 x int8).  A pair of blocks is 68 bytes =
//   17 dwords, so pairs start 4-byte aligned whatever the block parity; a lane
//   owns one pair (64 columns) per step: y += d0 * sum q*x + d1 * sum q*x.
// Q4_K: 144-byte super-blocks (fp16 d, dmin, 12 scale bytes, 128 nibble bytes).
//   A lane owns one quarter (qs bytes 32c..32c+31 = sub-blocks 2c and 2c+1,
//   64 columns) and reads the 16-byte header beside it; in factored form
//   y += d*(sc_lo*sum q_lo*x + sc_hi*sum q_hi*x) - dmin*(m_lo*sum x + m_hi*sum x),
//   where the sums of x depend only on the lane's columns and are computed once.
#include "qw35_device.h"
#include "qw35_kernels.h"

namespace qw35 {
namespace {

typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

// a*x staged as fp32 in LDS: xs[b*k + col].
template <int NB>
__device__ __forceinline__ void stage_x_f32(const float* __restrict__ x, const float* __restrict__ awq, int k,
                                            int n_batch, float* xs) {
    const int q4 = k >> 2;
    for (int i = threadIdx.x; i < q4; i += 256) {
        const float4_t a = awq ? *reinterpret_cast<const float4_t*>(awq + 4 * i) : float4_t{1.f, 1.f, 1.f, 1.f};
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float4_t v = {0.f, 0.f, 0.f, 0.f};
            if (b < n_batch) v = *reinterpret_cast<const float4_t*>(x + (size_t)b * k + 4 * i) * a;
            *reinterpret_cast<float4_t*>(xs + (size_t)b * k + 4 * i) = v;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ float byte_s8(uint32_t w, int byte) {
    return (float)(int32_t)(int8_t)(uint8_t)(w >> (8 * byte));
}

__device__ __forceinline__ float half_lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)w); }
__device__ __forceinline__ float half_hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }

// ---------------------------------------------------------------- q8_0
// NB batch rows, P pair-steps per lane per row, RW rows per wave; a 256-thread
// workgroup covers 4*RW rows (one wave per RW rows, the whole K per wave).
template <int NB, int P, int RW, bool SWIGLU>
__global__ __launch_bounds__(256) void q8_0_gemv_kernel(GemvArgs args) {
    extern __shared__ float xs[];
    constexpr int NM = SWIGLU ? 2 : 1;
    const int k = args.k;
    const int rows = args.rows;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + wave) * RW;
    const int pairs = k >> 6;
    const size_t row_bytes = (size_t)(k >> 5) * 34;

    uint32_t wv[NM][RW][P][17];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const uint8_t* wb = static_cast<const uint8_t*>(m == 0 ? args.w : args.w_up);
#pragma unroll
        for (int r = 0; r < RW; ++r) {
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const int p = j * 64 + lane;
                const int row = row0 + r;
                if (row < rows && p < pairs) {
                    const uint32_t* src = reinterpret_cast<const uint32_t*>(wb + (size_t)row * row_bytes + (size_t)p * 68);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const u32x4_a4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a4*>(src) + q);
                        wv[m][r][j][4 * q + 0] = v.x;
                        wv[m][r][j][4 * q + 1] = v.y;
                        wv[m][r][j][4 * q + 2] = v.z;
                        wv[m][r][j][4 * q + 3] = v.w;
                    }
                    wv[m][r][j][16] = __builtin_nontemporal_load(src + 16);
                } else {
#pragma unroll
                    for (int q = 0; q < 17; ++q) wv[m][r][j][q] = 0u;
                }
            }
        }
    }

    stage_x_f32<NB>(args.x, args.awq, k, args.n_batch, xs);

    float acc[NM][RW][NB];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[m][r][b] = 0.0f;

#pragma unroll
    for (int j = 0; j < P; ++j) {
        const int p = j * 64 + lane;
        if (p >= pairs) continue;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float* xp = xs + (size_t)b * k + 64 * p;
            float xv[64];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float4_t v = *reinterpret_cast<const float4_t*>(xp + 4 * i);
                xv[4 * i + 0] = v.x;
                xv[4 * i + 1] = v.y;
                xv[4 * i + 2] = v.z;
                xv[4 * i + 3] = v.w;
            }
#pragma unroll
            for (int m = 0; m < NM; ++m) {
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    const uint32_t* d = wv[m][r][j];
                    float s0 = 0.0f, s1 = 0.0f;
                    // block 0: qs at bytes 2..33 of the pair
#pragma unroll
                    for (int i = 0; i < 32; ++i) s0 = __builtin_fmaf(byte_s8(d[(2 + i) >> 2], (2 + i) & 3), xv[i], s0);
                    // block 1: qs at bytes 36..67
#pragma unroll
                    for (int i = 0; i < 32; ++i) s1 = __builtin_fmaf(byte_s8(d[9 + (i >> 2)], i & 3), xv[32 + i], s1);
                    acc[m][r][b] = __builtin_fmaf(half_lo(d[0]), s0, acc[m][r][b]);
                    acc[m][r][b] = __builtin_fmaf(half_hi(d[8]), s1, acc[m][r][b]);
                }
            }
        }
    }

#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[m][r][b] = wave_sum_to_lane63(acc[m][r][b]);
    if (lane == 63) {
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const int row = row0 + r;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (row < rows && b < args.n_batch) {
                    float* yp = args.y + (size_t)b * rows + row;
                    float v = SWIGLU ? silu(acc[0][r][b]) * acc[NM - 1][r][b] : acc[0][r][b];
                    if (args.residual) v += *yp;
                    *yp = v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------- Q4_K
// A lane owns quarter (blk, c) = (q / 4, q % 4) of quarter index q = j*64+lane.
template <int NB, int P, int RW, bool SWIGLU>
__global__ __launch_bounds__(256) void q4_k_gemv_kernel(GemvArgs args) {
    extern __shared__ float xs[];
    constexpr int NM = SWIGLU ? 2 : 1;
    const int k = args.k;
    const int rows = args.rows;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + wave) * RW;
    const int quarters = k >> 6;
    const size_t row_bytes = (size_t)(k >> 8) * 144;

    uint4_t hdr[NM][RW][P];
    uint4_t qv[NM][RW][P][2];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const uint8_t* wb = static_cast<const uint8_t*>(m == 0 ? args.w : args.w_up);
#pragma unroll
        for (int r = 0; r < RW; ++r) {
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const int q = j * 64 + lane;
                const int row = row0 + r;
                if (row < rows && q < quarters) {
                    const uint8_t* blk = wb + (size_t)row * row_bytes + (size_t)(q >> 2) * 144;
                    hdr[m][r][j] = *reinterpret_cast<const uint4_t*>(blk);
                    qv[m][r][j][0] = load_stream16(blk + 16 + 32 * (q & 3));
                    qv[m][r][j][1] = load_stream16(blk + 32 + 32 * (q & 3));
                } else {
                    hdr[m][r][j] = uint4_t{0u, 0u, 0u, 0u};
                    qv[m][r][j][0] = uint4_t{0u, 0u, 0u, 0u};
                    qv[m][r][j][1] = uint4_t{0u, 0u, 0u, 0u};
                }
            }
        }
    }

    stage_x_f32<NB>(args.x, args.awq, k, args.n_batch, xs);

    float acc[NM][RW][NB];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[m][r][b] = 0.0f;

#pragma unroll
    for (int j = 0; j < P; ++j) {
        const int q = j * 64 + lane;
        if (q >= quarters) continue;
        const int c = q & 3;
        const int col0 = (q >> 2) * 256 + 64 * c;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float* xp = xs + (size_t)b * k + col0;
            float xv[64];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float4_t v = *reinterpret_cast<const float4_t*>(xp + 4 * i);
                xv[4 * i + 0] = v.x;
                xv[4 * i + 1] = v.y;
                xv[4 * i + 2] = v.z;
                xv[4 * i + 3] = v.w;
            }
            float sx_lo = 0.0f, sx_hi = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                sx_lo += xv[i];
                sx_hi += xv[32 + i];
            }
#pragma unroll
            for (int m = 0; m < NM; ++m) {
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    const uint4_t h = hdr[m][r][j];
                    const uint32_t qw[8] = {qv[m][r][j][0].x, qv[m][r][j][0].y, qv[m][r][j][0].z, qv[m][r][j][0].w,
                                            qv[m][r][j][1].x, qv[m][r][j][1].y, qv[m][r][j][1].z, qv[m][r][j][1].w};
                    float sq_lo = 0.0f, sq_hi = 0.0f;
#pragma unroll
                    for (int i = 0; i < 32; ++i) {
                        const uint32_t byte = (qw[i >> 2] >> (8 * (i & 3))) & 0xFFu;
                        sq_lo = __builtin_fmaf((float)(byte & 0x0Fu), xv[i], sq_lo);
                        sq_hi = __builtin_fmaf((float)(byte >> 4), xv[32 + i], sq_hi);
                    }
                    // 6-bit scales/mins of sub-blocks 2c and 2c+1 (qw35_types.metal:70-83).
                    const uint32_t sb[12] = {h.y & 0xFF, (h.y >> 8) & 0xFF, (h.y >> 16) & 0xFF, h.y >> 24,
                                             h.z & 0xFF, (h.z >> 8) & 0xFF, (h.z >> 16) & 0xFF, h.z >> 24,
                                             h.w & 0xFF, (h.w >> 8) & 0xFF, (h.w >> 16) & 0xFF, h.w >> 24};
                    uint32_t sc0, m0, sc1, m1;
                    const int j0 = 2 * c, j1 = 2 * c + 1;
                    if (c < 2) {
                        sc0 = sb[j0] & 63; m0 = sb[j0 + 4] & 63;
                        sc1 = sb[j1] & 63; m1 = sb[j1 + 4] & 63;
                    } else {
                        sc0 = (sb[j0 + 4] & 0x0F) | ((sb[j0 - 4] >> 6) << 4);
                        m0 = (sb[j0 + 4] >> 4) | ((sb[j0] >> 6) << 4);
                        sc1 = (sb[j1 + 4] & 0x0F) | ((sb[j1 - 4] >> 6) << 4);
                        m1 = (sb[j1 + 4] >> 4) | ((sb[j1] >> 6) << 4);
                    }
                    const float d = half_lo(h.x);
                    const float dmin = half_hi(h.x);
                    const float qpart = (float)sc0 * sq_lo + (float)sc1 * sq_hi;
                    const float mpart = (float)m0 * sx_lo + (float)m1 * sx_hi;
                    acc[m][r][b] = __builtin_fmaf(d, qpart, acc[m][r][b]);
                    acc[m][r][b] = __builtin_fmaf(-dmin, mpart, acc[m][r][b]);
                }
            }
        }
    }

#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[m][r][b] = wave_sum_to_lane63(acc[m][r][b]);
    if (lane == 63) {
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const int row = row0 + r;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (row < rows && b < args.n_batch) {
                    float* yp = args.y + (size_t)b * rows + row;
                    float v = SWIGLU ? silu(acc[0][r][b]) * acc[NM - 1][r][b] : acc[0][r][b];
                    if (args.residual) v += *yp;
                    *yp = v;
                }
            }
        }
    }
}

int batch_slice_f32(int k) {
    const int budget = 48 * 1024;
    const int per_row = k * 4;
    if (4 * per_row <= budget) return 4;
    if (2 * per_row <= budget) return 2;
    return 1;
}

#define QW35_LAUNCH_KQ(KERNEL, NB, P, RW, SW)                                                          \
    do {                                                                                               \
        const int grid = (s.rows + 4 * (RW) - 1) / (4 * (RW));                                         \
        const size_t lds = (size_t)(NB) * s.k * sizeof(float);                                         \
        hipLaunchKernelGGL((KERNEL<NB, P, RW, SW>), dim3(grid), dim3(256), lds, stream, s);            \
        e = hipGetLastError();                                                                         \
    } while (0)

template <bool SW>
hipError_t launch_q8_0_any(const GemvArgs& a, hipStream_t stream) {
    const int slice = batch_slice_f32(a.k);
    for (int b0 = 0; b0 < a.n_batch; b0 += slice) {
        GemvArgs s = a;
        s.n_batch = a.n_batch - b0 < slice ? a.n_batch - b0 : slice;
        s.x = a.x + (size_t)b0 * a.k;
        s.y = a.y + (size_t)b0 * a.rows;
        hipError_t e = hipSuccess;
        const int pairs = a.k >> 6;
        const int P = (pairs + 63) / 64;
        if (s.n_batch == 1) {
            if (P <= 1) QW35_LAUNCH_KQ(q8_0_gemv_kernel, 1, 1, 2, SW);
            else if (P <= 2) QW35_LAUNCH_KQ(q8_0_gemv_kernel, 1, 2, 1, SW);
            else if (P <= 3) QW35_LAUNCH_KQ(q8_0_gemv_kernel, 1, 3, 1, SW);
            else QW35_LAUNCH_KQ(q8_0_gemv_kernel, 1, 8, 1, SW);
        } else if (s.n_batch == 2) {
            if (P <= 1) QW35_LAUNCH_KQ(q8_0_gemv_kernel, 2, 1, 1, SW);
            else if (P <= 2) QW35_LAUNCH_KQ(q8_0_gemv_kernel, 2, 2, 1, SW);
            else if (P <= 3) QW35_LAUNCH_KQ(q8_0_gemv_kernel, 2, 3, 1, SW);
            else QW35_LAUNCH_KQ(q8_0_gemv_kernel, 2, 8, 1, SW);
        } else {
            if (P <= 1) QW35_LAUNCH_KQ(q8_0_gemv_kernel, 4, 1, 1, SW);
            else if (P <= 2) QW35_LAUNCH_KQ(q8_0_gemv_kernel, 4, 2, 1, SW);
            else if (P <= 3) QW35_LAUNCH_KQ(q8_0_gemv_kernel, 4, 3, 1, SW);
            else QW35_LAUNCH_KQ(q8_0_gemv_kernel, 4, 8, 1, SW);
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <bool SW>
hipError_t launch_q4_k_any(const GemvArgs& a, hipStream_t stream) {
    const int slice = batch_slice_f32(a.k);
    for (int b0 = 0; b0 < a.n_batch; b0 += slice) {
        GemvArgs s = a;
        s.n_batch = a.n_batch - b0 < slice ? a.n_batch - b0 : slice;
        s.x = a.x + (size_t)b0 * a.k;
        s.y = a.y + (size_t)b0 * a.rows;
        hipError_t e = hipSuccess;
        const int quarters = a.k >> 6;
        const int P = (quarters + 63) / 64;
        if (s.n_batch == 1) {
            if (P <= 1) QW35_LAUNCH_KQ(q4_k_gemv_kernel, 1, 1, 2, SW);
            else if (P <= 2) QW35_LAUNCH_KQ(q4_k_gemv_kernel, 1, 2, 1, SW);
            else if (P <= 3) QW35_LAUNCH_KQ(q4_k_gemv_kernel, 1, 3, 1, SW);
            else QW35_LAUNCH_KQ(q4_k_gemv_kernel, 1, 8, 1, SW);
        } else if (s.n_batch == 2) {
            if (P <= 1) QW35_LAUNCH_KQ(q4_k_gemv_kernel, 2, 1, 1, SW);
            else if (P <= 2) QW35_LAUNCH_KQ(q4_k_gemv_kernel, 2, 2, 1, SW);
            else if (P <= 3) QW35_LAUNCH_KQ(q4_k_gemv_kernel, 2, 3, 1, SW);
            else QW35_LAUNCH_KQ(q4_k_gemv_kernel, 2, 8, 1, SW);
        } else {
            if (P <= 1) QW35_LAUNCH_KQ(q4_k_gemv_kernel, 4, 1, 1, SW);
            else if (P <= 2) QW35_LAUNCH_KQ(q4_k_gemv_kernel, 4, 2, 1, SW);
            else if (P <= 3) QW35_LAUNCH_KQ(q4_k_gemv_kernel, 4, 3, 1, SW);
            else QW35_LAUNCH_KQ(q4_k_gemv_kernel, 4, 8, 1, SW);
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_q8_0_gemv(const GemvArgs& a, hipStream_t stream) {
    return a.w_up ? launch_q8_0_any<true>(a, stream) : launch_q8_0_any<false>(a, stream);
}

hipError_t launch_q4_k_gemv(const GemvArgs& a, hipStream_t stream) {
    return a.w_up ? launch_q4_k_any<true>(a, stream) : launch_q4_k_any<false>(a, stream);
}

}  // namespace qw35
