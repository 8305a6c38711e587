// GF4 decode GEMV / fused gate-up-SwiGLU for gfx950, batch 1..8, on MFMA.
//
//   y[b][r] (+)= sum_k W[r][k] * a[k] * x[b][k]
//
// Weight format (GGUF type 100): one uint32 per 8 columns, bits 0..7 an e5m2
// scale byte, bits 8+3i..10+3i the code c_i = q_i ^ 4 of column 8g+i; the
// weight is (4 - q_i) * s / 4 (tools/qw35_cook_common.py:67-80,115-119).
// Reference kernels replaced: qw35_decode_matmul_gf4_2row{,_residual}_f32 and
// qw35_ffn_gate_up_swiglu_gf4_f32 (qw35-server/src/metal/qw35_gf4.metal:62-136,209-246).
//
// Mapping onto v_mfma_f32_16x16x32_f16 (D[16x16] += A[16x32] * B[32x16]):
//   * B = weights: lane l holds 8 consecutive k of weight row n = l % 16, i.e.
//     exactly one GF4 word, decoded in registers to exact fp16 values;
//   * A = activations: row m = 2b holds fp16(x_b) ("hi"), row 2b+1 holds
//     fp16(x_b - hi) ("lo"), so batch 1..8 fill the 16 A rows and the fp16
//     split keeps ~22 bits of each fp32 activation;
//   * D: lane l holds D[4*(l/16)+j][l%16]; y[b][n] = D[2b][n] + D[2b+1][n].
//
// Word -> 8 exact fp16 weights, 17 VALU ops:
//   t  = w ^ 0x92492400                  (q_i = c_i ^ 4 for the eight codes)
//   t1 = t >> 4, t2 = t >> 10
//   P0 = (t1 & 0x00070070) | 0x64005400  fp16 pair (64 + q0, 1024 + q4)
//   P1 = (t1 & 0x00380380) | 0x58004800  fp16 pair ( 8 + q1,  128 + q5)
//   P2 = (t2 & 0x00070070) | 0x64005400  fp16 pair (64 + q2, 1024 + q6)
//   P3 = (t2 & 0x00380380) | 0x58004800  fp16 pair ( 8 + q3,  128 + q7)
//   E_j = P_j - (base + 4)               exact small integers q - 4
//   B_j = E_j * (-s/4)                   exact: |q-4| <= 4 and s has 3 significant bits
// The pairs hold columns (0,4) (1,5) (2,6) (3,7); A is stored in LDS in the
// same order, which the MFMA's sum over k does not see.
//
// Activations are staged once per workgroup in LDS, scaled per batch row by a
// power of two that puts max|a*x| in [2^13, 2^14) (no fp16 overflow for any
// input magnitude); the factor is divided out exactly at the end.
//
// Launch: one workgroup per 16-row tile, KS waves splitting K, each wave
// covering CPW chunks of 256 columns (two 16-byte loads per lane per chunk).
// Every x load is issued before the weight loads, so waiting for x never waits
// on the weight stream (vector loads complete in order); the weights are then
// consumed in issue order as they arrive.
#include "gf4_decode.h"
#include "qw35_device.h"
#include "qw35_kernels.h"

#include <stdio.h>

#include <type_traits>

namespace qw35 {
namespace {

// s_waitcnt encoding (gfx9): wait until at most `n` vector-memory operations
// of this wave are outstanding; expcnt and lgkmcnt are left unconstrained.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Per-wave LDS block:
//   xpose    2 x 2 KB transpose buffers (16 rows x 128 bytes = one 256-column
//            chunk of a 16-row tile).  Global loads read full 128-byte lines
//            (lane l of instruction h: row 8h + l/8, 16-byte segment l%8); each
//            lane stores its segment s of row r at r*128 + 16*(s ^ ((r>>1)&7)),
//            and the MFMA-layout reads (row n, segments 2kq and 2kq+1) then hit
//            16 distinct bank groups per 16 lanes.
//   acts     2*NB rows (hi, lo of each batch row) x (CPW*256 + 8) halves, each
//            group of 8 columns stored as x0 x4 x1 x5 x2 x6 x3 x7.
//   zeros    64 halves (the A operand of rows past the batch).
// After the KS blocks: the per-wave partial outputs.
template <int NB, int CPW, bool BD = false>
struct WaveLds {
    static constexpr int kXposeBytes = 2 * 2048;
    static constexpr int kStride = CPW * 256 + 8;  // halves per activation row
    static constexpr int kActBytes = 2 * NB * kStride * 2;
    static constexpr int kXwOff = kXposeBytes + kActBytes + 128;
    static constexpr int kXwBytes = BD ? NB * CPW * 32 * 4 : 0;  // per-word bias sums (block-diagonal form)
    static constexpr int kBytes = kXwOff + kXwBytes;
};

template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (N > 0) {
        static_for<N - 1>(f);
        f(std::integral_constant<int, N - 1>{});
    }
}

// Workgroup = KS waves covering 16*RT rows x all k.  Wave w owns the K-slice
// [w*CPW*256, (w+1)*CPW*256) of all RT row tiles; its weight loads are issued
// up front in the order (chunk, tile, matrix, half) and consumed in that order.
//
// BD (block-diagonal form, batch 1..2): A row 4j+i holds the activations of
// word j of the MFMA's four words only (i = 0,1: hi, lo of batch row 0;
// i = 2,3: of batch row 1), so D[4j+i][n] is the partial of one word of row n,
// and it lands in the lane that decoded that word.  B is then the biased
// decode P = base + q (6 VALU ops, gf4_word_to_biased) and the word's scale is
// applied once in fp32:
//   sum_i (4 - q_i) x_i * s/4 = (s/4) * (X''_w - D_hi - D_lo),
//   X''_w = sum_i (4 + base_i) * x_i    (row-independent, staged with the activations).
template <int NB, int RT, int KS, int CPW, bool SWIGLU, bool HAS_AWQ, bool BD>
__global__ __launch_bounds__(64 * KS) void gf4_mfma_gemv(GemvArgs args) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int NM = SWIGLU ? 2 : 1;
    static_assert(!BD || NB <= 2, "block-diagonal form holds two batch rows");
    using L = WaveLds<NB, CPW, BD>;
    constexpr int STRIDE = L::kStride;
    constexpr int GPL = (CPW * 32 + 63) / 64;  // activation groups per lane per batch row
    constexpr int NTC = CPW * RT * NM;         // tile-chunks per wave
    constexpr int NLOADS = 2 * NTC;
    constexpr int NKQ = BD ? 4 : 1;            // lane groups holding distinct partials
    static_assert(NLOADS <= 48, "vmcnt budget");
    const int k = args.k;
    const int rows = args.rows;
    const int n_batch = args.n_batch;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 15;
    const int kq = lane >> 4;
    const int row0 = blockIdx.x * 16 * RT;
    const int words_per_row = k >> 3;
    const int col0 = wave * CPW * 256;
    const int slice_groups = min(CPW * 32, max(0, (k - col0) >> 3));

    uint8_t* wblk = smem + (size_t)wave * L::kBytes;
    _Float16* xs = reinterpret_cast<_Float16*>(wblk + L::kXposeBytes);
    _Float16* zrow = xs + 2 * NB * STRIDE;
    float* xw = reinterpret_cast<float*>(wblk + L::kXwOff);                  // [NB][CPW*32] (BD)
    float* part = reinterpret_cast<float*>(smem + (size_t)KS * L::kBytes);  // [KS][RT][NM][NB][NKQ][16]
    if (lane < 32) reinterpret_cast<uint32_t*>(zrow)[lane] = 0u;

    // 1. Activation slice (and AWQ) into registers, clamped, unused until step 3.
    float4_t xv[NB][GPL][2];
    float4_t av[GPL][2];
#pragma unroll
    for (int j = 0; j < GPL; ++j) {
        int g = lane + 64 * j;
        g = g < slice_groups ? g : 0;
        const int col = col0 + 8 * g;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int bb = b < n_batch ? b : 0;
            const float* src = args.x + (size_t)bb * k + col;
            xv[b][j][0] = *reinterpret_cast<const float4_t*>(src);
            xv[b][j][1] = *reinterpret_cast<const float4_t*>(src + 4);
        }
        if (HAS_AWQ) {
            av[j][0] = *reinterpret_cast<const float4_t*>(args.awq + col);
            av[j][1] = *reinterpret_cast<const float4_t*>(args.awq + col + 4);
        }
    }

    // Keep the scheduler from sinking the activation loads below the weight
    // loads: vector loads complete in order, so waiting for x must not wait
    // for the weight stream.
    __builtin_amdgcn_sched_barrier(0);

    // 2. Weight loads, full 128-byte lines per 8 lanes.  Rows past the end are
    //    clamped (computed on a duplicate row, never stored).
    uint4_t wv[NTC][2];
    const int lrow = lane >> 3;  // row within the half tile
    const int lseg = lane & 7;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        int chunk = wave * CPW + c;
        chunk = chunk * 256 < k ? chunk : 0;
#pragma unroll
        for (int t = 0; t < RT; ++t) {
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const uint32_t* wbase = static_cast<const uint32_t*>(m == 0 ? args.w : args.w_up);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    int r = row0 + 16 * t + 8 * h + lrow;
                    r = r < rows ? r : rows - 1;
                    wv[(c * RT + t) * NM + m][h] =
                        load_stream16(wbase + (size_t)r * words_per_row + chunk * 32 + 4 * lseg);
                }
            }
        }
    }

    __builtin_amdgcn_sched_barrier(0);

    // 3. Wave-private fp16 hi/lo activations with a per-wave power-of-two scale
    //    (and, BD, the per-word bias sums X'' of the same hi + lo values).
    wait_vmcnt<NLOADS>();
    float inv_scale[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        float mx = 0.0f;
#pragma unroll
        for (int j = 0; j < GPL; ++j) {
            if (HAS_AWQ) {
                xv[b][j][0] *= av[j][0];
                xv[b][j][1] *= av[j][1];
            }
            if (lane + 64 * j < slice_groups) {
#pragma unroll
                for (int e = 0; e < 4; ++e) mx = fmaxf(mx, fmaxf(fabsf(xv[b][j][0][e]), fabsf(xv[b][j][1][e])));
            }
        }
        const float sc = fp16_range_scale(wave_max_abs(mx));
        inv_scale[b] = pow2_inverse(sc);
#pragma unroll
        for (int j = 0; j < GPL; ++j) {
            const int g = lane + 64 * j;
            if (g < slice_groups) {
                const float4_t v0 = xv[b][j][0] * sc;
                const float4_t v1 = xv[b][j][1] * sc;
                const float e[8] = {v0[0], v1[0], v0[1], v1[1], v0[2], v1[2], v0[3], v1[3]};
                uint32_t hi[4], lo[4];
                float xsum = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const half2_t hh = h2(e[2 * q], e[2 * q + 1]);
                    const half2_t ll = h2(e[2 * q] - (float)hh.x, e[2 * q + 1] - (float)hh.y);
                    hi[q] = as_u32(hh);
                    lo[q] = as_u32(ll);
                    if constexpr (BD) {
                        xsum = __builtin_fmaf(gf4_bias(2 * q), (float)hh.x + (float)ll.x, xsum);
                        xsum = __builtin_fmaf(gf4_bias(2 * q + 1), (float)hh.y + (float)ll.y, xsum);
                    }
                }
                *reinterpret_cast<uint4_t*>(xs + (size_t)(2 * b) * STRIDE + 8 * g) = uint4_t{hi[0], hi[1], hi[2], hi[3]};
                *reinterpret_cast<uint4_t*>(xs + (size_t)(2 * b + 1) * STRIDE + 8 * g) =
                    uint4_t{lo[0], lo[1], lo[2], lo[3]};
                if constexpr (BD) xw[b * CPW * 32 + g] = xsum;
            }
        }
    }

    // 4. Per tile-chunk: transpose through LDS, decode, MFMA.  All LDS data
    //    here is private to the wave and LDS operations of one wave execute in
    //    order, so no workgroup barrier is needed before the compute.
    const int mrow = lane & 15;
    // A operand row of this lane: plain form, rows 2b / 2b+1 of the batch;
    // BD form, row 4j+i carries word j == kq only.
    const bool a_live = BD ? ((mrow >> 2) == kq && ((mrow & 3) >> 1) < n_batch) : (mrow < 2 * n_batch);
    const _Float16* arow = xs + (size_t)(BD ? (mrow & 3) : mrow) * STRIDE + 64 * kq;
    const int swz_r = (n >> 1) & 7;
    const int rd0 = n * 128 + 16 * ((2 * kq) ^ swz_r);
    const int rd1 = n * 128 + 16 * ((2 * kq + 1) ^ swz_r);
    const int wr0 = lrow * 128 + 16 * (lseg ^ ((lrow >> 1) & 7));              // h = 0: rows 0..7
    const int wr1 = (8 + lrow) * 128 + 16 * (lseg ^ (((8 + lrow) >> 1) & 7));  // h = 1: rows 8..15
    const Gf4Consts cst = gf4_consts();
    float4_t acc[RT][NM];   // plain form: the D accumulator
    float accb[RT][NM][2];  // BD form: batch rows 0, 1 of word partials of this lane group
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            acc[t][m] = float4_t{0.f, 0.f, 0.f, 0.f};
            accb[t][m][0] = accb[t][m][1] = 0.0f;
        }
    half8_t a[8];
    float xwv[NB][8];

    static_for<NTC>([&](auto I) {
        constexpr int i = decltype(I)::value;
        constexpr int c = i / (RT * NM);
        constexpr int t = (i / NM) % RT;
        constexpr int m = i % NM;
        if ((wave * CPW + c) * 256 < k) {
            if constexpr (t == 0 && m == 0) {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const _Float16* ap = a_live ? arow + c * 256 : zrow;
#pragma unroll
                for (int q = 0; q < 8; ++q) a[q] = *reinterpret_cast<const half8_t*>(ap + (a_live ? 8 * q : 0));
                if constexpr (BD) {
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        const float4_t u0 = *reinterpret_cast<const float4_t*>(xw + b * CPW * 32 + c * 32 + 8 * kq);
                        const float4_t u1 = *reinterpret_cast<const float4_t*>(xw + b * CPW * 32 + c * 32 + 8 * kq + 4);
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            xwv[b][q] = u0[q];
                            xwv[b][4 + q] = u1[q];
                        }
                    }
                }
            }
            wait_vmcnt<NLOADS - 2 * (i + 1)>();
            uint8_t* xb = wblk + (i & 1) * 2048;
            *reinterpret_cast<uint4_t*>(xb + wr0) = wv[i][0];
            *reinterpret_cast<uint4_t*>(xb + wr1) = wv[i][1];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const uint4_t w0 = *reinterpret_cast<const uint4_t*>(xb + rd0);
            const uint4_t w1 = *reinterpret_cast<const uint4_t*>(xb + rd1);
            const uint32_t ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            if constexpr (BD) {
                // All eight MFMAs first (independent, zero accumulator), so the
                // fp32 epilogues do not wait on each MFMA's latency.
                float4_t dd[8];
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    dd[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[q], gf4_word_to_biased(ww[q], cst),
                                                                   float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float s = gf4_scale_f32(ww[q]);
                    accb[t][m][0] = __builtin_fmaf(s, (xwv[0][q] - dd[q][0]) - dd[q][1], accb[t][m][0]);
                    if constexpr (NB == 2)
                        accb[t][m][1] = __builtin_fmaf(s, (xwv[NB - 1][q] - dd[q][2]) - dd[q][3], accb[t][m][1]);
                }
                // Schedule: decode of word q (6 VALU) then its MFMA, eight times,
                // then the epilogues.
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    acc[t][m] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(a[q], gf4_word_to_b(ww[q], cst), acc[t][m], 0, 0, 0);
            }
        }
    });

    // 5. Per-wave partials, scaled back by the wave's activation scale, into
    //    LDS and summed over the KS waves (and, BD, the four lane groups).
    //    Plain form: lane group kq holds batches 2kq and 2kq+1 (D rows 4kq..4kq+3).
    if constexpr (BD) {
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    part[((((wave * RT + t) * NM + m) * NB + b) * 4 + kq) * 16 + n] =
                        accb[t][m][b] * (0.25f * inv_scale[b]);
    } else {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
#pragma unroll
            for (int m = 0; m < NM; ++m) {
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const int b = 2 * kq + jj;
                    float isc = 1.0f;
#pragma unroll
                    for (int bb = 0; bb < NB; ++bb)
                        if (bb == b) isc = inv_scale[bb];
                    if (b < NB)
                        part[(((wave * RT + t) * NM + m) * NB + b) * 16 + n] =
                            (acc[t][m][2 * jj] + acc[t][m][2 * jj + 1]) * isc;
                }
            }
        }
    }
    __syncthreads();
    for (int o = threadIdx.x; o < RT * NB * 16; o += 64 * KS) {
        const int t = o / (NB * 16);
        const int b = (o / 16) % NB;
        const int nn = o & 15;
        const int r = row0 + 16 * t + nn;
        float tot[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < KS; ++w)
#pragma unroll
                for (int g = 0; g < NKQ; ++g) sum += part[((((w * RT + t) * NM + m) * NB + b) * NKQ + g) * 16 + nn];
            tot[m] = sum;
        }
        if (r < rows && b < n_batch) {
            float* yp = args.y + (size_t)b * rows + r;
            float v = SWIGLU ? silu(tot[0]) * tot[NM - 1] : tot[0];
            if (args.residual) v += *yp;
            *yp = v;
        }
    }
}

// Largest batch of the block-diagonal form (0 disables it).
#ifndef QW35_GF4_BD_MAX_BATCH
#define QW35_GF4_BD_MAX_BATCH 2
#endif

template <int NB, int RT, int KS, int CPW, bool SWIGLU, bool BD>
size_t lds_bytes() {
    constexpr int NM = SWIGLU ? 2 : 1;
    return (size_t)KS * WaveLds<NB, CPW, BD>::kBytes + (size_t)KS * RT * NM * NB * (BD ? 4 : 1) * 16 * 4;
}

template <int NB, int RT, int KS, int CPW, bool SWIGLU>
hipError_t launch_cfg(const GemvArgs& a, hipStream_t stream) {
    constexpr bool BD = NB <= QW35_GF4_BD_MAX_BATCH;
    const size_t lds = lds_bytes<NB, RT, KS, CPW, SWIGLU, BD>();
    if (lds > 160 * 1024) return hipErrorInvalidConfiguration;
    if ((a.k >> 8) > KS * CPW) return hipErrorInvalidValue;  // every chunk belongs to a wave
    const int grid = (a.rows + 16 * RT - 1) / (16 * RT);
    if (a.info) {
        snprintf(a.info->name, sizeof a.info->name, "gf4_mfma_gemv<%d, %d, %d, %d, %s, %s, %s>", NB, RT, KS, CPW,
                 SWIGLU ? "true" : "false", a.awq ? "true" : "false", BD ? "true" : "false");
        a.info->grid = (unsigned)grid;
        a.info->block = 64u * KS;
        a.info->lds = (unsigned)lds;
        return hipSuccess;
    }
    if (a.awq) {
        hipLaunchKernelGGL((gf4_mfma_gemv<NB, RT, KS, CPW, SWIGLU, true, BD>), dim3(grid), dim3(64 * KS), lds, stream,
                           a);
    } else {
        hipLaunchKernelGGL((gf4_mfma_gemv<NB, RT, KS, CPW, SWIGLU, false, BD>), dim3(grid), dim3(64 * KS), lds, stream,
                           a);
    }
    return hipGetLastError();
}

// Launch plan for a shape: KS waves per workgroup, CPW 256-column chunks per
// wave (KS*CPW*256 >= k), RT 16-row tiles per workgroup.  RT is raised for
// tall matrices so that one workgroup per CU re-reads the activations once
// for 48 rows instead of 16.
struct Gf4Plan {
    int rt, ks, cpw;
};

// Shapes measured on MI355X (graph replays over 805 MB of rotated weights):
// 12288 x 4096 b1 {3, 8, 2} 7.10 us; fused gate/up b1 {3, 16, 1} 11.6 us
// ({3, 8, 2} 12.2 us); 4096 x 12288 b1 {1, 12, 4} 8.01 us ({1, 8, 6} 8.41 us).
Gf4Plan plan_gf4(int nb, int rows, int k, bool swiglu) {
    const int chunks = k / 256;
    const int tiles = (rows + 15) / 16;
    if (chunks <= 4) return {1, 4, 1};
    if (chunks <= 8) return {1, 4, 2};
    if (chunks <= 16) {
        if (tiles >= 768) return (swiglu && nb == 1) ? Gf4Plan{3, 16, 1} : Gf4Plan{3, 8, 2};
        if (tiles >= 512) return {2, 8, 2};
        return {1, 8, 2};
    }
    if (chunks <= 32) return {1, 8, 4};
    if (chunks <= 48 && nb == 1) return {1, 12, 4};
    return {1, 8, 6};
}

size_t plan_lds(const Gf4Plan& p, int nb, bool swiglu) {
    const int nm = swiglu ? 2 : 1;
    const bool bd = nb <= QW35_GF4_BD_MAX_BATCH;
    const size_t per_wave = 4096 + (size_t)2 * nb * (p.cpw * 256 + 8) * 2 + 128 + (bd ? (size_t)nb * p.cpw * 32 * 4 : 0);
    return (size_t)p.ks * per_wave + (size_t)p.ks * p.rt * nm * nb * (bd ? 4 : 1) * 16 * 4;
}

template <int NB, bool SWIGLU>
hipError_t launch_nb(const GemvArgs& a, hipStream_t stream) {
    const Gf4Plan p = plan_gf4(NB, a.rows, a.k, SWIGLU);
#define QW35_GF4_PLAN(RT, KS, CPW) \
    if (p.rt == RT && p.ks == KS && p.cpw == CPW) return launch_cfg<NB, RT, KS, CPW, SWIGLU>(a, stream);
    QW35_GF4_PLAN(1, 4, 1)
    QW35_GF4_PLAN(1, 4, 2)
    QW35_GF4_PLAN(1, 8, 2)
    QW35_GF4_PLAN(2, 8, 2)
    QW35_GF4_PLAN(3, 8, 2)
    if constexpr (NB <= 4) { QW35_GF4_PLAN(1, 8, 4) }
    if constexpr (NB <= 2) { QW35_GF4_PLAN(1, 8, 6) }
    if constexpr (NB == 1) {
        QW35_GF4_PLAN(3, 16, 1)
        QW35_GF4_PLAN(1, 12, 4)
    }
#undef QW35_GF4_PLAN
    return hipErrorInvalidValue;
}

// Largest batch slice (8, 4, 2, 1 rows) whose plan fits the 160 KiB LDS.
int gf4_batch_slice(const GemvArgs& a, bool swiglu) {
    int slice = 8;
    while (slice > 1 && plan_lds(plan_gf4(slice, a.rows, a.k, swiglu), slice, swiglu) > 160 * 1024) slice >>= 1;
    return slice;
}

template <bool SWIGLU>
hipError_t launch_gf4_any(const GemvArgs& a, hipStream_t stream) {
    const int slice = gf4_batch_slice(a, SWIGLU);
    if (plan_lds(plan_gf4(1, a.rows, a.k, SWIGLU), 1, SWIGLU) > 160 * 1024) return hipErrorInvalidValue;
    for (int b0 = 0; b0 < a.n_batch; b0 += slice) {
        GemvArgs s = a;
        s.n_batch = a.n_batch - b0 < slice ? a.n_batch - b0 : slice;
        s.x = a.x + (size_t)b0 * a.k;
        s.y = a.y + (size_t)b0 * a.rows;
        hipError_t e;
        if (s.n_batch == 1) e = launch_nb<1, SWIGLU>(s, stream);
        else if (s.n_batch == 2) e = launch_nb<2, SWIGLU>(s, stream);
        else if (s.n_batch <= 4) e = launch_nb<4, SWIGLU>(s, stream);
        else e = launch_nb<8, SWIGLU>(s, stream);
        if (e != hipSuccess) return e;
        if (a.info) break;  // describe the first slice's launch only
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_gf4_gemv(const GemvArgs& a, hipStream_t stream) {
    // When the activations of the whole batch do not fit this kernel's LDS it
    // would stream the weights once per batch slice; the chunked kernel (per-chunk
    // activation staging) takes the batch in one launch.  It also takes k beyond
    // 48 chunks (12288), which no plan of this kernel covers.
    if ((a.k >> 8) > 48 || a.n_batch > gf4_batch_slice(a, a.w_up != nullptr))
        return launch_gf4_gemv_chunked(a, stream);
    return a.w_up ? launch_gf4_any<true>(a, stream) : launch_gf4_any<false>(a, stream);
}

}  // namespace qw35
