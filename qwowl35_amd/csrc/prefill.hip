// Prefill dequant-matmul on MFMA (gfx950): the tiled multi-token matmul of
// encodeMatvecBatch / encodeTiledKMatmul
// (qw35-server/src/metal/bridge/Qw35MetalRuntime+FFN.m:260-366; kernels
// qw35_mul_mm_gf4_f32 / qw35_kernel_mul_mm in qw35_tiled_mm.metal:36-255):
//
//   C[m][n] = sum_k v[m][k] * W[n][k],  v = awq[k] * A[m][k] (fp32), fp32 accumulation,
//
// A: [M][K] bf16 or fp32 activations, W: [N][K] weights, C: [M][N] bf16 (RNE) or
// fp32 (STORE, or the ADD / SwiGLU epilogues of the runtime's chunk).
//
// * Staged path (the default; the caller passes a workspace):
//   prefill_stage_kernel writes v as fp16 with a per-token power-of-two scale
//   (fp32 input: an fp16 hi and lo row per token, ~22 significant bits), and
//   gf4_prefill_f16_kernel contracts it on v_mfma_f32_32x32x16_f16 against the
//   weights decoded in registers: GF4 words (exact in fp16), q8_0 blocks and
//   Q4_K super-blocks dequantised in the kernel to fp16 of their exact value,
//   or F16 weights (the fp16 prefill image of the other k-quants).  Tiles,
//   K halves / quarters within a block and K splits across blocks (fp32
//   partial sums, prefill_split_reduce) follow plan_prefill.  A launch may
//   cover up to kMaxSegments matrices over the same activations (a mixer's
//   input projections), and a GF4 gate/up pair as one fused launch.
// * Direct path (GF4, bf16 activations without AWQ, no workspace):
//   gf4_prefill_kernel stages A and the GF4 tile decoded to bf16 in LDS and
//   contracts on v_mfma_f32_16x16x32_bf16.  GF4 decode is exact in bf16 and
//   fp16: w_i = -sext3(c_i) * s / 4, s = fp16(b << 8) (the format of
//   tools/qw35_cook_common.py:79 with c = q_raw ^ 4).
// * Blocks are assigned XCD by XCD (consecutive block ids land on different
//   XCDs), so the blocks that share a weight tile share an L2.
#include <stdio.h>

#include <cmath>
#include <type_traits>

#include "gf4_decode.h"
#include "qw35_device.h"
#include "qw35_kernels.h"

namespace qw35 {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

constexpr int kBK = 64;                 // k per pipeline step: 8 GF4 words per W row
constexpr int kLdsRow = kBK * 2 + 16;   // bytes per staged row: 64 bf16 + 16 B pad
// Token-tile LDS buffers per K part of the staged kernel: four (a barrier
// every second step) for tiles of up to 128 staged rows, two (a barrier every
// step) for the 256-row tiles, whose register allocation is at its limit.
template <int BM>
constexpr int token_buffers() { return BM <= 128 ? 4 : 2; }
constexpr int kXcds = 8;

struct PrefillArgs {
    const uint32_t* w;       // GF4 words [N][K/8]
    const void* a;           // [M][K] bf16 or fp32 (staged path: fp16, see below)
    const float* awq;        // [K] or nullptr
    void* c;                 // [M][N] bf16 or fp32
    const float* row_scale;  // staged path: per token, the inverse of its fp16 scale
    int m, n, k;             // m: rows of a (staged path: staged rows)
    int m_out;               // rows of c (tokens)
    int hilo;                // staged fp32 input: MFMA tiles 2i, 2i + 1 are one token tile's hi, lo rows
    int epi;                 // fp32 c: kEpiStore c = r, kEpiAdd c += r, kEpiSwiglu c = silu(c) * r
    LaunchInfo* info;        // host pointer: describe the matmul launch here instead of launching
    int tiles_m, tiles_n;
    int splits;              // staged path: K split this many ways (1: none)
    int k_len;               // columns per split
    // Staged path, n_seg > 1: up to kMaxSegments matrices over the same
    // activations in one launch.  Segment s has seg_n[s] rows, its weights at
    // seg_w[s] and its own output seg_c[s] ([m_out][seg_n[s]]); its blocks are
    // the seg_tiles[s] weight tiles after those of the segments before it.
    // Split launches write the partial sums of all segments as one
    // [m_out][n] array (n = the sum of seg_n), segment s at column seg_col[s].
    int n_seg;
    int seg_n[kMaxSegments], seg_col[kMaxSegments], seg_tiles[kMaxSegments];
    const void* seg_w[kMaxSegments];
    void* seg_c[kMaxSegments];
    // Fused gate/up (GF4 words, staged path, no split): the up projection's
    // words; c = silu(gate) * up.
    const uint32_t* w_up;
};

// How a result r is written to fp32 c.
constexpr int kEpiStore = 0, kEpiAdd = 1, kEpiSwiglu = 2;

__device__ __forceinline__ float epilogue(int epi, float old, float r) {
    return epi == kEpiAdd ? old + r : epi == kEpiSwiglu ? silu(old) * r : r;
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{lo, hi}, bf16x2_t));
}

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __builtin_bit_cast(float, v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __builtin_bit_cast(float, v & 0xFFFF0000u); }

// One GF4 word -> its 8 weights as bf16 (exact).
__device__ __forceinline__ uint4_t gf4_word_to_bf16x8(uint32_t w) {
    const float ns4 = (float)__builtin_bit_cast(_Float16, (uint16_t)(w << 8)) * -0.25f;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)(int)__builtin_amdgcn_sbfe((int)w, 8 + 3 * i, 3) * ns4;
    return uint4_t{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7])};
}

// Staged activations (the path taken when the caller provides a workspace).
// v = awq * A in fp32 (A read exactly from bf16 or fp32; awq == nullptr:
// v = A), and 2^e the power of two that puts the token row's max |v| in
// [2^14, 2^15); row_scale = 2^-e.
// * bf16 input: one staged fp16 row per token, fp16_rne(2^e v).  Without AWQ
//   every bf16 value of at least 2^-28 of the row maximum is exact (smaller
//   ones round at 2^-39 of the maximum); with AWQ the product is rounded once,
//   to fp16 (11 significant bits).
// * fp32 input (HILO): two staged fp16 rows per token, hi = fp16_rne(2^e v)
//   and lo = fp16_rne((2^e v - hi) 2^11) (the difference is exact in fp32), so
//   hi + 2^-11 lo carries about 22 significant bits of v: the activations
//   keep fp32 precision, as the reference's tiled matmul keeps src1 in fp32
//   (qw35-server/src/metal/qw35_tiled_mm.metal:200-224).  Token t's rows are
//   64 (t / 32) + t % 32 (hi) and that + 32 (lo): in a block of staged rows
//   the 32-row MFMA tiles 2i and 2i + 1 hold the same 32 tokens' hi and lo
//   halves, and the matmul adds their accumulators (hi + 2^-11 lo) before the
//   row scale.  The grid covers tokens 0 .. 32 ceil(M / 32) - 1; the padding
//   tokens' rows are written as zeros.
// The fp16 values feed fp16 MFMA with the weights decoded by the 15-op fp16
// GF4 decode of gf4_decode.h (or fp16 q8_0 / F16 weights).  Each group of 8
// columns is stored in the decode's column order 0,4,1,5,2,6,3,7 (GF4_ORDER),
// or in column order for the F16 and q8_0 weight kernels.
// 512 threads per token row: one staging launch (m = 128, fp32) took 2.79 us
// against 2.87 with 256 threads at k = 4096 and 4.35 against 4.62 at
// k = 12288 (same box, back-to-back launches); behind the matmuls of a
// prefill call or chunk the difference stays within 0.5%.
constexpr int kStageThreads = 512;

// G: groups of 8 columns each thread keeps in registers between the two
// passes (ceil(k / 4096), at most 6: k <= 24576); every one of its loads is
// issued before the first is used (an index past the row re-reads the row's
// last group and is left out of the maximum and the stores), so a thread
// waits for one load latency, not G in turn.  Longer rows read the rest again
// for the second pass.
template <bool A_F32, bool HAS_AWQ, bool GF4_ORDER, int G>
__global__ __launch_bounds__(kStageThreads) void prefill_stage_kernel(const void* __restrict__ a,
                                                                      const float* __restrict__ awq, int m, int k,
                                                                      uint16_t* __restrict__ a16,
                                                                      float* __restrict__ row_scale) {
    constexpr bool HILO = A_F32;
    const int row = blockIdx.x;
    const int groups = k >> 3;
    const size_t hi_row = HILO ? (size_t)64 * (row >> 5) + (row & 31) : (size_t)row;
    uint16_t* const dst_hi = a16 + hi_row * k;
    uint16_t* const dst_lo = dst_hi + (size_t)32 * k;
    if (HILO && row >= m) {  // padding token: zero rows, never stored by the matmul
        for (int g = threadIdx.x; g < groups; g += kStageThreads) {
            *reinterpret_cast<uint4_t*>(dst_hi + 8 * g) = uint4_t{0u, 0u, 0u, 0u};
            *reinterpret_cast<uint4_t*>(dst_lo + 8 * g) = uint4_t{0u, 0u, 0u, 0u};
        }
        return;
    }
    // v = awq * A of columns 8g..8g+7, fp32
    auto load8 = [&](int g, float (&o)[8]) {
        const size_t e0 = (size_t)row * k + 8 * g;
        if constexpr (A_F32) {
            const float4_t lo = *reinterpret_cast<const float4_t*>(static_cast<const float*>(a) + e0);
            const float4_t hi = *reinterpret_cast<const float4_t*>(static_cast<const float*>(a) + e0 + 4);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                o[q] = lo[q];
                o[4 + q] = hi[q];
            }
        } else {
            const uint4_t u = *reinterpret_cast<const uint4_t*>(static_cast<const uint16_t*>(a) + e0);
            const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                o[2 * q] = bf16_lo(w4[q]);
                o[2 * q + 1] = bf16_hi(w4[q]);
            }
        }
        if constexpr (HAS_AWQ) {
            const float4_t s0 = *reinterpret_cast<const float4_t*>(awq + 8 * g);
            const float4_t s1 = *reinterpret_cast<const float4_t*>(awq + 8 * g + 4);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                o[q] *= s0[q];
                o[4 + q] *= s1[q];
            }
        }
    };
    float v[G][8];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const int g = threadIdx.x + j * kStageThreads;
        load8(g < groups ? g : groups - 1, v[j]);
    }
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < G; ++j) {
        float mj = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q) mj = fmaxf(mj, fabsf(v[j][q]));
        if (threadIdx.x + j * kStageThreads < groups) mx = fmaxf(mx, mj);
    }
    for (int g = threadIdx.x + G * kStageThreads; g < groups; g += kStageThreads) {
        float t[8];
        load8(g, t);
#pragma unroll
        for (int q = 0; q < 8; ++q) mx = fmaxf(mx, fabsf(t[q]));
    }
    __shared__ float red[kStageThreads / 64];
    mx = wave_max_abs(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < kStageThreads / 64; ++w) mx = fmaxf(mx, red[w]);
    const float sc = 2.0f * fp16_range_scale(mx);  // max in [2^14, 2^15)
    if (threadIdx.x == 0) row_scale[row] = pow2_inverse(sc);
    // the 8 values of a group in storage order, as 4 packed pairs
    auto pack = [&](const float (&x)[8]) -> uint4_t {
        return GF4_ORDER ? uint4_t{as_u32(h2(x[0], x[4])), as_u32(h2(x[1], x[5])), as_u32(h2(x[2], x[6])),
                                   as_u32(h2(x[3], x[7]))}
                         : uint4_t{as_u32(h2(x[0], x[1])), as_u32(h2(x[2], x[3])), as_u32(h2(x[4], x[5])),
                                   as_u32(h2(x[6], x[7]))};
    };
    auto store8 = [&](int g, const float (&x)[8]) {
        float s[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) s[q] = x[q] * sc;
        *reinterpret_cast<uint4_t*>(dst_hi + 8 * g) = pack(s);
        if constexpr (HILO) {
            float r[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) r[q] = (s[q] - (float)(_Float16)s[q]) * 2048.0f;
            *reinterpret_cast<uint4_t*>(dst_lo + 8 * g) = pack(r);
        }
    };
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const int g = threadIdx.x + j * kStageThreads;
        if (g < groups) store8(g, v[j]);
    }
    for (int g = threadIdx.x + G * kStageThreads; g < groups; g += kStageThreads) {
        float t[8];
        load8(g, t);
        store8(g, t);
    }
}

// The staging launch: G from k (groups of 8 columns per thread held in registers).
template <bool A_F32, bool HAS_AWQ, bool GF4_ORDER>
void launch_stage(unsigned grid, hipStream_t stream, const void* a, const float* awq, int m, int k, uint16_t* a16,
                  float* rs) {
    const int g = (k / 8 + kStageThreads - 1) / kStageThreads;
#define QW35_STAGE_G(GG)                                                                                        \
    hipLaunchKernelGGL((prefill_stage_kernel<A_F32, HAS_AWQ, GF4_ORDER, GG>), dim3(grid), dim3(kStageThreads), 0, \
                       stream, a, awq, m, k, a16, rs)
    switch (g <= 1 ? 1 : g >= 6 ? 6 : g) {
        case 1: QW35_STAGE_G(1); break;
        case 2: QW35_STAGE_G(2); break;
        case 3: QW35_STAGE_G(3); break;
        case 4: QW35_STAGE_G(4); break;
        case 5: QW35_STAGE_G(5); break;
        default: QW35_STAGE_G(6); break;
    }
#undef QW35_STAGE_G
}

// Staged rows for m tokens: one per token, or (fp32 input) a hi and a lo row
// per token padded to whole 32-token groups.
inline int staged_rows(int m, bool a_f32) { return a_f32 ? 64 * ((m + 31) / 32) : m; }

template <int BM, int BN, int NT, bool A_F32>
struct StepRegs {
    static constexpr int A_CHUNKS = BM * 8 / NT;  // 8-element A chunks per thread
    static constexpr int WPT = BN * 8 / NT;       // GF4 words per thread
    uint4_t a[A_CHUNKS][A_F32 ? 2 : 1];
    uint32_t b[WPT];
};

// Direct path: bf16 MFMA on A' converted in the loader.
// Two waves per SIMD (<= 256 VGPRs): one wave's loads and conversions overlap
// the other's MFMAs.
template <int BM, int BN, int WGM, int WGN, bool A_F32, bool HAS_AWQ, bool OUT_F32>
__global__ __launch_bounds__(64 * WGM * WGN) __attribute__((amdgpu_waves_per_eu(2))) void gf4_prefill_kernel(
    PrefillArgs p) {
    constexpr int NT = 64 * WGM * WGN;
    constexpr int WTM = BM / WGM;      // wave tile (tokens)
    constexpr int WTN = BN / WGN;      // wave tile (weight rows)
    constexpr int FM = WTM / 16;       // MFMA tiles per wave
    constexpr int FN = WTN / 16;
    using Regs = StepRegs<BM, BN, NT, A_F32>;
    constexpr int A_CHUNKS = Regs::A_CHUNKS;
    constexpr int WPT = Regs::WPT;
    constexpr int BUF = (BM + BN) * kLdsRow;
    static_assert(BM * 8 % NT == 0 && A_CHUNKS >= 1, "A tile must split evenly over the threads");
    static_assert(BN * 8 % NT == 0 && (WPT == 1 || WPT == 2 || WPT == 4), "W tile must split into 1/2/4 words");
    static_assert(FM >= 1 && FN >= 1 && WTM % 16 == 0 && WTN % 16 == 0, "wave tile shape");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WGN;
    const int wn = wave % WGN;

    // XCD-major tile order, M-tile fastest within an XCD's share.
    const int tiles = p.tiles_m * p.tiles_n;
    int t = blockIdx.x;
    if (tiles % kXcds == 0) t = (t % kXcds) * (tiles / kXcds) + t / kXcds;
    const int m0 = (t % p.tiles_m) * BM;
    const int n0 = (t / p.tiles_m) * BN;
    const int K = p.k;
    const int words_per_row = K >> 3;
    const Gf4Consts gc = gf4_consts();

    // Per-thread global sources (rows clamped into range; stores are masked).
    const uint8_t* a_src[A_CHUNKS];
    int a_lds[A_CHUNKS];
    int a_col[A_CHUNKS];
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
        const int c = tid + i * NT;
        const int row = c >> 3;
        const int col = c & 7;
        const int gm = min(m0 + row, p.m - 1);
        a_src[i] = static_cast<const uint8_t*>(p.a) + ((size_t)gm * K + col * 8) * (A_F32 ? 4 : 2);
        a_lds[i] = row * kLdsRow + col * 16;
        a_col[i] = col * 8;
    }
    const int b_row = (tid * WPT) >> 3;
    const int b_g0 = (tid * WPT) & 7;
    const uint32_t* b_src = p.w + (size_t)min(n0 + b_row, p.n - 1) * words_per_row + b_g0;
    const int b_lds = BM * kLdsRow + b_row * kLdsRow + b_g0 * 16;

    auto load_step = [&](int kt, Regs& r) {
        const int k0 = kt * kBK;
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            if constexpr (A_F32) {
                r.a[i][0] = *reinterpret_cast<const uint4_t*>(a_src[i] + (size_t)k0 * 4);
                r.a[i][1] = *reinterpret_cast<const uint4_t*>(a_src[i] + (size_t)k0 * 4 + 16);
            } else {
                r.a[i][0] = *reinterpret_cast<const uint4_t*>(a_src[i] + (size_t)k0 * 2);
            }
        }
        const uint32_t* bs = b_src + (k0 >> 3);
        if constexpr (WPT == 4) {
            const uint4_t v = load_cached16(bs);
            r.b[0] = v.x; r.b[1] = v.y; r.b[2] = v.z; r.b[3] = v.w;
        } else if constexpr (WPT == 2) {
            typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));
            const uint2_t v = __builtin_nontemporal_load(reinterpret_cast<const uint2_t*>(bs));
            r.b[0] = v.x; r.b[1] = v.y;
        } else {
            r.b[0] = __builtin_nontemporal_load(bs);
        }
    };

    auto store_step = [&](int kt, const Regs& r, uint8_t* buf) {
        const int k0 = kt * kBK;
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            uint4_t out;
            if constexpr (!A_F32 && !HAS_AWQ) {
                out = r.a[i][0];
            } else {
                float v[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // element copies first: bit_cast of a vector-element lvalue reads element 0
                    const uint32_t e0 = r.a[i][0][j];
                    if constexpr (A_F32) {
                        const uint32_t e1 = r.a[i][1][j];
                        v[j] = __builtin_bit_cast(float, e0);
                        v[4 + j] = __builtin_bit_cast(float, e1);
                    } else {
                        v[2 * j] = bf16_lo(e0);
                        v[2 * j + 1] = bf16_hi(e0);
                    }
                }
                if constexpr (HAS_AWQ) {
                    const float4_t s0 = *reinterpret_cast<const float4_t*>(p.awq + k0 + a_col[i]);
                    const float4_t s1 = *reinterpret_cast<const float4_t*>(p.awq + k0 + a_col[i] + 4);
                    v[0] *= s0.x; v[1] *= s0.y; v[2] *= s0.z; v[3] *= s0.w;
                    v[4] *= s1.x; v[5] *= s1.y; v[6] *= s1.z; v[7] *= s1.w;
                }
                out = uint4_t{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]),
                              pack_bf16(v[6], v[7])};
            }
            *reinterpret_cast<uint4_t*>(buf + a_lds[i]) = out;
        }
#pragma unroll
        for (int q = 0; q < WPT; ++q)
            *reinterpret_cast<uint4_t*>(buf + b_lds + q * 16) = gf4_word_to_bf16x8(r.b[q]);
    };

    // The W tile is the MFMA's first operand and the token tile its second, so
    // lane l accumulates D[n = 4*(l/16) + r][m = l % 16]: four consecutive
    // outputs of one token row, written as one vector.
    float4_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    const int a_rd = (wm * WTM + (lane & 15)) * kLdsRow + (lane >> 4) * 16;
    const int b_rd = BM * kLdsRow + (wn * WTN + (lane & 15)) * kLdsRow + (lane >> 4) * 16;

    auto compute = [&](const uint8_t* cur) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            bf16x8_t af[FM], wf[FN];
#pragma unroll
            for (int j = 0; j < FN; ++j)
                wf[j] = *reinterpret_cast<const bf16x8_t*>(cur + b_rd + j * 16 * kLdsRow + ks * 64);
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *reinterpret_cast<const bf16x8_t*>(cur + a_rd + i * 16 * kLdsRow + ks * 64);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[j], af[i], acc[i][j], 0, 0, 0);
        }
    };

    // Two register stages: step kt+2 is loaded while step kt is contracted and
    // step kt+1 (loaded one step earlier) is converted into the other buffer.
    const int KT = K / kBK;
    uint8_t* buf0 = smem;
    uint8_t* buf1 = smem + BUF;
    Regs r0, r1;
    load_step(0, r0);
    if (KT > 1) load_step(1, r1);
    store_step(0, r0, buf0);
    __syncthreads();
    for (int kt = 0; kt < KT; kt += 2) {
        if (kt + 2 < KT) load_step(kt + 2, r0);
        compute(buf0);
        if (kt + 1 < KT) store_step(kt + 1, r1, buf1);
        __syncthreads();
        if (kt + 1 >= KT) break;
        if (kt + 3 < KT) load_step(kt + 3, r1);
        compute(buf1);
        if (kt + 2 < KT) store_step(kt + 2, r0, buf0);
        __syncthreads();
    }

    const bool vec_ok = (p.n & 3) == 0;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int gm = m0 + wm * WTM + i * 16 + (lane & 15);
        if (gm >= p.m) continue;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int gn = n0 + wn * WTN + j * 16 + (lane >> 4) * 4;
            const size_t o = (size_t)gm * p.n + gn;
            const float4_t d = acc[i][j];
            if (vec_ok && gn + 3 < p.n) {
                if constexpr (OUT_F32) {
                    *reinterpret_cast<float4_t*>(static_cast<float*>(p.c) + o) = d;
                } else {
                    typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));
                    *reinterpret_cast<uint2_t*>(static_cast<uint16_t*>(p.c) + o) =
                        uint2_t{pack_bf16(d.x, d.y), pack_bf16(d.z, d.w)};
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (gn + r < p.n) {
                        if constexpr (OUT_F32)
                            static_cast<float*>(p.c)[o + r] = d[r];
                        else
                            static_cast<uint16_t*>(p.c)[o + r] = (uint16_t)pack_bf16(d[r], 0.0f);
                    }
                }
            }
        }
    }
}

// Staged path: fp16 A'' (prefill_stage_kernel) against GF4 words decoded
// straight from global memory into MFMA operand registers.
//
// * A block owns a BM x (32 * FN * NW) tile of C.  Its NW waves split the
//   weight rows (32 * FN per wave) and all read the block's BM token rows from
//   LDS, so every
//   GF4 word is loaded and decoded (15 VALU ops, fp16, gf4_decode.h) by exactly
//   one wave and the only LDS traffic is the token tile.
// * v_mfma_f32_32x32x16_f16 with the weight tile as first operand: lane l
//   supplies weight row l % 32 and receives D[n][m = l % 32], four consecutive
//   weight rows per register group, so results leave as 8- or 16-byte stores.
// * Within a 64-wide k step lane half h of sub-step kk takes the 8 columns of
//   GF4 word 4h + kk, so each lane's four words of a row are one 16-byte load;
//   the token operand follows that order (and the decode's 0,4,1,5,2,6,3,7
//   column order, which the staging pass already wrote).
// * Global loads run two steps ahead in two register stages; the token tile
//   is double buffered in LDS, one barrier per step.
// * F16W: the weights are an fp16 tensor [N][K] (the prefill image of a
//   k-quant projection) instead of GF4 words.  A lane's 32 columns of a step
//   are four 16-byte loads, each the MFMA operand of one sub-step as it is:
//   no decode, and the token tile is staged in column order.
// * Q8W: the weights are q8_0 blocks (34 bytes: fp16 d, 32 int8 q) read and
//   dequantised in the kernel, no image.  A step (64 columns) is two blocks
//   of each row; lane half h takes block h, 8 columns per sub-step, in column
//   order like F16W.  The lane's 34 bytes start 4-byte aligned (h = 0) or 2
//   past it (h = 1); it loads the 16-byte aligned 48 bytes around its 36-byte
//   span (the span's dword offset in them, kt mod 4, is static in the
//   four-step loop body; at the last step of a range it is 3, so nothing past
//   the range is read) and realigns with v_perm.  B = fp16(d * q): the int8
//   to exact fp16 of the decode GEMVs, then one v_pk_mul_f16 by (d, d) -- the
//   same bits as the F16 prefill image, fp16_rne(d * q).
// * Q4W: the weights are Q4_K super-blocks (144 bytes per 256 columns: fp16 d
//   and dmin, 12 bytes of 6-bit sub-block scales and mins, 128 bytes of
//   nibbles) dequantised in the kernel, as the reference's tiled matmul does
//   (qw35_mul_mm_q4_k_f32, qw35_tiled_mm.metal:209-214), no image.  A step's
//   64 columns are the sub-block pair 2j, 2j + 1 (j = kt mod 4) of each row,
//   whose elements are the low and high nibbles of the same 32 bytes
//   qs[32j .. 32j + 31]; lane half h takes sub-block 2j + h, 8 columns per
//   sub-step in column order.  A lane loads the super-block's 16-byte header
//   and the 32 bytes (three 16-byte loads; the header line stays cached for
//   the four steps of a super-block).  B = fp16_rne(fl32(d sc q - dmin m)):
//   d sc and dmin m are exact fp32 products formed once per step, one fma per
//   weight rounds once -- the exact dequantised value of
//   qw35_dequant_q4_k_at (qw35_matvec.metal:2-12), then the same fp16 bits as
//   the F16 prefill image.
// * SWI (fused gate/up, GF4 words, FN = 2): tile 0 of a wave is 32 rows of the
//   gate projection and tile 1 the same rows of the up projection (p.w_up);
//   the epilogue writes silu(g) * u, g and u each the fp32 value the gate
//   launch (STORE) and the up launch (SWIGLU epilogue) of the same plan would
//   form -- the same K partition and MFMA order per tile, so the same bits.
//   FN = 1 (mixed tiles): a wave's one tile holds 16 rows of the gate (rows
//   0..15) and the same 16 rows of the up projection (rows 16..31); a lane's
//   accumulators hold rows 8 g + 4 h + r, so gate row c and up row c pair up
//   in the same lane (g and g + 2).  A block then covers 16 rows per wave of
//   a K part, e.g. 96 rows on 6 waves: 12288 rows in 128 column tiles.
template <int BM, int NW, int FN, int WPE, bool OUT_F32, bool F16W = false, bool Q8W = false, int KH = 1,
          bool Q4W = false, bool SWI = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void gf4_prefill_f16_kernel(
    PrefillArgs p) {
    static_assert(!SWI || ((FN == 1 || FN == 2) && OUT_F32 && !F16W && !Q8W && !Q4W),
                  "fused gate/up: GF4 words, a gate and an up tile per wave or one mixed tile");
    constexpr bool MIX = SWI && FN == 1;    // one tile of 16 gate and 16 up rows per wave
    constexpr int NWG = NW / KH;            // waves per K half
    constexpr int NTG = 64 * NWG;           // threads per K half
    constexpr int TPW = SWI ? 1 : FN;       // distinct 32-row output tiles per wave
    constexpr int BN = (MIX ? 16 : 32 * TPW) * NWG;  // output rows (columns of C) per block
    constexpr int FM = BM / 32;             // 32-token MFMA tiles per wave; FN: 32-row weight tiles per wave
    // 16-byte token chunks per thread per step: BM * 8 over the part's
    // threads, the last one only where the split is uneven (three waves per part)
    constexpr int A_ALL = BM * 8;
    constexpr int A_CHUNKS = (A_ALL + NTG - 1) / NTG;
    constexpr int BUF = BM * kLdsRow;
    static_assert(BM % 32 == 0 && A_CHUNKS >= 1, "token tile rows in whole MFMA tiles");
    static_assert((KH == 1 || KH == 2 || KH == 4) && NW % KH == 0, "one, two or four K parts of equal wave counts");
    // (the fused gate/up kernel hands its gate and up sums over in two passes)
    static_assert(KH == 1 || (KH / 2) * NWG * FM * (SWI ? 1 : FN) * 16 * 64 * 4 <= token_buffers<BM>() * KH * BUF,
                  "K-part partial sums fit the token buffers");
    typedef float float16_t __attribute__((ext_vector_type(16)));
    typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = lane >> 5;
    const int l32 = lane & 31;

    // Block -> (split, tile): the blocks of one K range are consecutive, and
    // the XCD remap hands each XCD a contiguous run of them.
    const int tiles = p.tiles_m * p.tiles_n;
    const int blocks = tiles * p.splits;
    int t = blockIdx.x;
    if (blocks % kXcds == 0) t = (t % kXcds) * (blocks / kXcds) + t / kXcds;
    const int split = t / tiles;
    t -= split * tiles;
    const int m0 = (t % p.tiles_m) * BM;
    // The block's matrix (uniform): its weights, rows, output and the output's
    // row stride and first column.
    int tn = t / p.tiles_m;
    const uint32_t* W = p.w;
    int N = p.n;
    void* C = p.c;
    int ld = p.n, col0 = 0;
    if (p.n_seg > 1) {
        int sg = 0;
        while (sg + 1 < p.n_seg && tn >= p.seg_tiles[sg]) {
            tn -= p.seg_tiles[sg];
            ++sg;
        }
        W = static_cast<const uint32_t*>(p.seg_w[sg]);
        N = p.seg_n[sg];
        if (p.splits > 1) {
            col0 = p.seg_col[sg];  // C: the partial sums of all segments, ld = p.n
        } else {
            C = p.seg_c[sg];
            ld = N;
        }
    }
    // KH = 2 (4): waves [kh NWG, (kh + 1) NWG) take part kh of the block's K
    // range, two halves (four quarters), over the same rows, each part with its
    // own token tile; the parts are summed in LDS at the end.
    const int kh = KH > 1 ? wave / NWG : 0;
    const int tg = tid - kh * NTG;
    const int n0 = tn * BN + (wave - kh * NWG) * (MIX ? 16 : 32 * TPW);
    const int K = p.k;
    const int k_len = p.k_len / KH;
    const int k_begin = split * p.k_len + kh * k_len;
    const int words_per_row = K >> 3;
    const Gf4Consts gc = gf4_consts();

    uint32_t a_off[A_CHUNKS];
    int a_lds[A_CHUNKS];
    // an uneven split: the last chunk of threads past the tile re-reads the
    // tile's last chunk and stores nothing
    const bool a_last = A_ALL % NTG == 0 || tg + (A_CHUNKS - 1) * NTG < A_ALL;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
        const int c = min(tg + i * NTG, A_ALL - 1);
        const int row = c >> 3;
        const int col = c & 7;
        const int gm = min(m0 + row, p.m - 1);
        a_off[i] = ((uint32_t)gm * (uint32_t)K + (uint32_t)k_begin + (uint32_t)col * 8u) * 2u;
        a_lds[i] = row * kLdsRow + col * 16;
    }
    constexpr int WCH = F16W ? 4 : (Q8W || Q4W) ? 3 : 1;  // 16-byte weight loads per lane per 32-row tile per step
    const uint8_t* w_src[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const size_t row = (size_t)min(n0 + (MIX ? (l32 & 15) : (SWI ? 0 : 32 * j) + l32), N - 1);
        if constexpr (Q4W)
            w_src[j] = reinterpret_cast<const uint8_t*>(W) + row * (size_t)(K / 256 * 144) + (k_begin / 256) * 144;
        else if constexpr (Q8W)
            w_src[j] = reinterpret_cast<const uint8_t*>(W) + row * (size_t)(K / 32 * 34) + (k_begin / 32) * 34 +
                       32 * half;
        else
            w_src[j] = F16W ? reinterpret_cast<const uint8_t*>(W) + (row * K + k_begin + 32 * half) * 2
                            : reinterpret_cast<const uint8_t*>(((MIX ? l32 >= 16 : SWI && j == 1) ? p.w_up : W) +
                                                               row * words_per_row +
                                                               (k_begin >> 3) + 4 * half);
    }
    // Q8W: byte selectors for this lane half (span dword i -> q dword i; d -> (d, d))
    const uint32_t q8_sel = half ? 0x07060504u : 0x05040302u;
    const uint32_t q8_dsel = half ? 0x03020302u : 0x01000100u;
    const half2_t q8_bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint8_t* a_base = static_cast<const uint8_t*>(p.a);

    typedef uint4_t Tokens[A_CHUNKS];
    typedef uint4_t Words[FN][WCH];
    auto load_tokens = [&](int kt, Tokens& a) {
        const uint32_t k0 = (uint32_t)kt * kBK;
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) a[i] = *reinterpret_cast<const uint4_t*>(a_base + a_off[i] + k0 * 2);
    };
    auto load_words = [&](int kt, Words& w) {
        const size_t k0 = (size_t)kt * kBK;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int c = 0; c < WCH; ++c)
                w[j][c] = load_cached16(w_src[j] + (Q4W   ? (k0 / 256) * 144 + (c ? 16 * c + 32 * ((k0 / 64) & 3) : 0)
                                                    : Q8W  ? (k0 / 64) * 68 - 4 * ((k0 / 64) & 3) + 16 * c
                                                    : F16W ? k0 * 2 + 16 * c
                                                           : k0 / 2));
    };
    auto store_tokens = [&](const Tokens& a, uint8_t* buf) {
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i)
            if (i + 1 < A_CHUNKS || a_last) *reinterpret_cast<uint4_t*>(buf + a_lds[i]) = a[i];
    };

    float16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    const int a_rd = l32 * kLdsRow + half * 64;

    // A step's four 16-k sub-steps run as a two-stage pipeline: the weight
    // decode and token-tile LDS reads of sub-step kk + 1 are issued between
    // the MFMAs of sub-step kk (explicit scheduling groups), so the decode
    // VALU and the LDS latency overlap the matrix pipe instead of preceding it.
    auto compute = [&](const Words& w, const uint8_t* buf, auto SPAN) {
        half8_t wf[2][FN], af[2][FM];
        // Q8W: the lane's span starts at dword kt mod 4 of its three loads
        constexpr int s0 = decltype(SPAN)::value;
        auto span = [&](int j, int i) -> uint32_t {
            const int d = s0 + i;
            const uint4_t v = w[j][d >> 2];
            return (d & 3) == 0 ? v.x : (d & 3) == 1 ? v.y : (d & 3) == 2 ? v.z : v.w;
        };
        // Q4W: the step's sub-block scale and min of this lane half, per tile
        // (sub-block 2 * (kt mod 4) + half, unpacked as get_scale_min_k4)
        float q4_dsc[FN], q4_dm[FN];
        if constexpr (Q4W) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const uint4_t hd = w[j][0];
                const half2_t dd = as_half2(hd.x);
                uint32_t sc, mn;
                if constexpr (s0 < 2) {  // sub-blocks 0..3: scales[sb] and scales[sb + 4], low 6 bits
                    const uint32_t sh = 8u * (2u * s0 + (uint32_t)half);
                    sc = (hd.y >> sh) & 63u;
                    mn = (hd.z >> sh) & 63u;
                } else {  // sub-blocks 4..7: low / high nibble of scales[sb + 4], top bits of scales[sb - 4] / [sb]
                    const uint32_t sh = 8u * (2u * (s0 - 2) + (uint32_t)half);
                    const uint32_t hi = hd.w >> sh;
                    sc = (hi & 0x0Fu) | (((hd.y >> sh) >> 6 & 3u) << 4);
                    mn = ((hi >> 4) & 0x0Fu) | (((hd.z >> sh) >> 6 & 3u) << 4);
                }
                q4_dsc[j] = (float)dd.x * (float)sc;
                q4_dm[j] = (float)dd.y * (float)mn;
            }
        }
        auto fetch = [&](int kk, int s) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                if constexpr (Q4W) {
                    // bytes 8kk .. 8kk + 7 of the pair's 32: loads 1 (bytes 0..15) and 2 (16..31)
                    const uint4_t v = w[j][1 + (kk >> 1)];
                    uint32_t q2[2] = {(kk & 1) ? v.z : v.x, (kk & 1) ? v.w : v.y};
                    float e[8];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t nib = (half ? q2[h] >> 4 : q2[h]) & 0x0F0F0F0Fu;
#pragma unroll
                        for (int b = 0; b < 4; ++b)  // v_cvt_f32_ubyte<b>; fp32 rounding, then fp16
                            e[4 * h + b] =
                                keep_f32(__builtin_fmaf(q4_dsc[j], (float)((nib >> (8 * b)) & 0xFFu), -q4_dm[j]));
                    }
                    wf[s][j] = __builtin_bit_cast(half8_t, uint4_t{as_u32(h2(e[0], e[1])), as_u32(h2(e[2], e[3])),
                                                                   as_u32(h2(e[4], e[5])), as_u32(h2(e[6], e[7]))});
                } else if constexpr (Q8W) {
                    const half2_t d2 = as_half2(__builtin_amdgcn_perm(span(j, 0), span(j, 0), q8_dsel));
                    uint32_t b[4];
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        const uint32_t qs = __builtin_amdgcn_perm(span(j, 2 * kk + q + 1), span(j, 2 * kk + q), q8_sel);
                        const uint32_t t = qs ^ 0x80808080u;  // q + 128 in each byte
                        b[2 * q] = as_u32((as_half2(__builtin_amdgcn_perm(0x64646464u, t, 0x04010400u)) + q8_bias) * d2);
                        b[2 * q + 1] =
                            as_u32((as_half2(__builtin_amdgcn_perm(0x64646464u, t, 0x04030402u)) + q8_bias) * d2);
                    }
                    wf[s][j] = __builtin_bit_cast(half8_t, uint4_t{b[0], b[1], b[2], b[3]});
                } else if constexpr (F16W) {
                    wf[s][j] = __builtin_bit_cast(half8_t, w[j][kk]);
                } else {
                    const uint32_t word = kk == 0 ? w[j][0].x : kk == 1 ? w[j][0].y : kk == 2 ? w[j][0].z : w[j][0].w;
                    wf[s][j] = gf4_word_to_b(word, gc);
                }
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[s][i] = *reinterpret_cast<const half8_t*>(buf + a_rd + i * 32 * kLdsRow + kk * 16);
        };
        if constexpr (Q8W) {
            // The span uses 9 of the 12 loaded dwords.  Keep all 12 live up to
            // here: a dword left dead would be reallocated while its load is
            // in flight, and that write-after-write makes the compiler wait
            // for every outstanding load, the prefetches of the next two
            // steps included (two full waits per four steps).
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int c = 0; c < WCH; ++c) asm volatile("" ::"v"(w[j][c]));
        }
        fetch(0, 0);
        // Sub-step 0's operands are issued before any MFMA, and each
        // sub-step's scheduling region then holds its MFMAs and the next one's
        // reads (GF4 12288x4096 M = 2048 211 -> 206 us; q8_0 8192x4096
        // M = 2048 174 -> 168 us)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int s = kk & 1;
            if (kk < 3) fetch(kk + 1, s ^ 1);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[s][j], af[s][i], acc[i][j], 0, 0, 0);
            if (kk < 3) {
                // per MFMA: one LDS read (the first FM of them) and a share of
                // the next sub-step's decode (15 VALU per word, FN words)
                constexpr int kValuPerMfma =
                    F16W ? 0 : ((Q4W ? 26 : Q8W ? 16 : 15) * FN + FM * FN - 1) / (FM * FN);
#pragma unroll
                for (int q = 0; q < FM * FN; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                    if (q < FM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                    if (kValuPerMfma > 0) __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);  // VALU
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Pipeline, per step kt: the step's weight words were loaded at step kt-2
    // into a four-slot register ring, and its tokens sit in an LDS buffer.  A
    // step first issues its prefetches (words into the ring slot two ahead,
    // tokens into the register set the previous step emptied into LDS), then
    // runs its MFMAs, then writes tokens loaded one step earlier to LDS.
    // * Two buffers (NBUF = 2): tokens of step kt+2 are loaded, those of kt+1
    //   written to the other buffer, and every step ends in a barrier.
    // * Four buffers: tokens of step kt+3 are loaded, those of kt+2 written to
    //   buffer (kt+2) mod 4, and a barrier ends every odd step.  A buffer is
    //   read two steps after it is written, and written two steps after it
    //   was last read, with a barrier between each pair.  Same-box A/B (us,
    //   two -> four, bit-identical): GF4 12288x4096 fp32 M = 128 42.1 ->
    //   40.3, 4096x12288 fp32 M = 48 29.5 -> 28.7, bf16 M = 2048 201 -> 197;
    //   the 9B 128-token chunk 6213 -> 6148.
    // The words ring and the loop body cover four steps, so every register
    // set is loaded and consumed under one static name and nothing loaded is
    // copied across the loop back-edge (a copy would wait for the load).  Each
    // split covers a multiple of 4 * kBK columns (the host checks k_len % 256
    // == 0); the prefetches past the last step re-read it instead of branching.
    constexpr int NBUF = token_buffers<BM>();
    static_assert(NBUF * KH * BUF <= 160 * 1024, "token buffers fit the CU's LDS");
    const int KT = k_len / kBK;
    uint8_t* const tbuf = smem + kh * NBUF * BUF;
    Tokens t0, t1;
    Words w0, w1, w2, w3;
    load_tokens(0, t0);
    load_words(0, w0);
    load_tokens(1, t1);
    load_words(1, w1);
    store_tokens(t0, tbuf);
    if constexpr (NBUF == 4) {
        store_tokens(t1, tbuf + BUF);
        load_tokens(min(2, KT - 1), t0);
    }
    __syncthreads();
    // SPAN: kt mod 4 (the unrolled position; Q8W's span offset and the buffer)
    auto step = [&](int kt, Tokens& t_next, Words& w_next, const Words& w_cur, const Tokens& t_fill, auto SPAN) {
        constexpr int s4 = decltype(SPAN)::value;
        load_tokens(min(kt + NBUF / 2 + 1, KT - 1), t_next);
        load_words(min(kt + 2, KT - 1), w_next);
        __builtin_amdgcn_sched_barrier(0);  // issue the prefetch before this step's math
        compute(w_cur, tbuf + (s4 % NBUF) * BUF, SPAN);
        store_tokens(t_fill, tbuf + ((s4 + NBUF / 2) % NBUF) * BUF);
        if constexpr (NBUF == 2 || s4 % 2 == 1)
            __syncthreads();
        else
            __builtin_amdgcn_sched_barrier(0);  // the step boundary stays a scheduling fence
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    for (int kt = 0; kt < KT; kt += 4) {
        if constexpr (NBUF == 4) {
            step(kt, t1, w2, w0, t0, S0{});
            step(kt + 1, t0, w3, w1, t1, S1{});
            step(kt + 2, t1, w0, w2, t0, S2{});
            step(kt + 3, t0, w1, w3, t1, S3{});
        } else {
            step(kt, t0, w2, w0, t1, S0{});
            step(kt + 1, t1, w3, w1, t0, S1{});
            step(kt + 2, t0, w0, w2, t1, S2{});
            step(kt + 3, t1, w1, w3, t0, S3{});
        }
    }

    if constexpr (KH > 1) {
        // Partial sums pass through LDS (free after the last step's barrier):
        // halves as (first + second); quarters as (q0 + q1) + (q2 + q3), the
        // odd quarters handing over to the even ones, then q2 to q0.  The same
        // order for every launch.
        constexpr int kPart = NWG * FM * FN * 16 * 64;  // floats of one part's sums
        float* xch = reinterpret_cast<float*>(smem) + (size_t)(wave - kh * NWG) * FM * FN * 16 * 64 + lane;
        auto put = [&](float* x) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) x[((i * FN + j) * 16 + r) * 64] = acc[i][j][r];
        };
        auto add = [&](const float* x) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] += x[((i * FN + j) * 16 + r) * 64];
        };
        if constexpr (SWI) {
            // the gate tiles, then the up tiles (one tile's sums per pass fit the
            // token buffers), each in the order of the unfused kernel
            constexpr int kPart1 = NWG * FM * 16 * 64;  // floats of one part's sums of one tile
            float* const x1 = reinterpret_cast<float*>(smem) + (size_t)(wave - kh * NWG) * FM * 16 * 64 + lane;
            auto put1 = [&](float* x, int j) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) x[(i * 16 + r) * 64] = acc[i][j][r];
            };
            auto add1 = [&](const float* x, int j) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] += x[(i * 16 + r) * 64];
            };
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                if constexpr (KH == 4) {
                    if (kh & 1) put1(x1 + (kh >> 1) * kPart1, j);
                    __syncthreads();
                    if (!(kh & 1)) add1(x1 + (kh >> 1) * kPart1, j);
                    __syncthreads();
                    if (kh == 2) put1(x1, j);
                    __syncthreads();
                    if (kh == 0) add1(x1, j);
                    __syncthreads();
                } else {
                    if (kh == 1) put1(x1, j);
                    __syncthreads();
                    if (kh == 0) add1(x1, j);
                    __syncthreads();
                }
            }
            if (kh != 0) return;
        } else if constexpr (KH == 4) {
            if (kh & 1) put(xch + (kh >> 1) * kPart);
            __syncthreads();
            if (!(kh & 1)) add(xch + (kh >> 1) * kPart);
            __syncthreads();
            if (kh == 2) put(xch);
            __syncthreads();
            if (kh != 0) return;
            add(xch);
        } else {
            if (kh == 1) put(xch);
            __syncthreads();
            if (kh == 1) return;
            add(xch);
        }
    }
    if constexpr (SWI) {
        // c = silu(g) * u: g and u as the gate launch stores them and the up
        // launch's SWIGLU epilogue forms them (the sums times the row scale)
        float* const cf = static_cast<float*>(C);
        const bool vec = (ld & 3) == 0 && ((uintptr_t)C & 15) == 0;
        auto put_row = [&](int gm, float rs, auto v_of) {
            // two tiles: row 8 g + 4 h + r of tile 0 (gate) and tile 1 (up);
            // mixed: that row (g < 2) and row 16 + that row of tile 0
#pragma unroll
            for (int g = 0; g < (MIX ? 2 : 4); ++g) {
                const int gn = n0 + 8 * g + 4 * half;
                float d[4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    d[r] = MIX ? epilogue(kEpiSwiglu, v_of(0, g, r) * rs, v_of(0, g + 2, r) * rs)
                               : epilogue(kEpiSwiglu, v_of(0, g, r) * rs, v_of(FN - 1, g, r) * rs);
                float* const dst = cf + (size_t)gm * ld + gn;
                if (vec && gn + 3 < N) {
                    *reinterpret_cast<float4_t*>(dst) = float4_t{d[0], d[1], d[2], d[3]};
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (gn + r < N) dst[r] = d[r];
                }
            }
        };
        if (p.hilo) {
            if constexpr (FM % 2 == 0) {
#pragma unroll
                for (int i = 0; i < FM / 2; ++i) {
                    const int gm = m0 / 2 + 32 * i + l32;
                    if (gm >= p.m_out) continue;
                    put_row(gm, p.row_scale[gm], [&](int j, int g, int r) {
                        return acc[2 * i][j][4 * g + r] + acc[2 * i + 1][j][4 * g + r] * 0x1p-11f;
                    });
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int gm = m0 + 32 * i + l32;
                if (gm >= p.m_out) continue;
                put_row(gm, p.row_scale[gm], [&](int j, int g, int r) { return acc[i][j][4 * g + r]; });
            }
        }
        return;
    }

    // Lane l holds D[n = 8 g + 4 h + r][m = l % 32] in acc[..][4 g + r].
    // Split launches write unscaled fp32 partial sums, split s at
    // c + s * m_out * n (OUT_F32 is then true); prefill_split_reduce finishes.
    void* const c = OUT_F32 ? static_cast<void*>(static_cast<float*>(C) + (size_t)split * p.m_out * ld + col0) : C;
    const bool vec_ok = (ld & 3) == 0 && (col0 & 3) == 0 && ((uintptr_t)C & 15) == 0;
    // split launches write partial sums; the reduction applies the epilogue
    const int epi = OUT_F32 && p.splits == 1 ? p.epi : kEpiStore;
    // token gm's 4 x 4 outputs of weight tile j: d(g, r) is row n0 + 32 j + 8 g + 4 half + r
    auto emit = [&](int gm, int j, float rs, auto d_of) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int gn = n0 + 32 * j + 8 * g + 4 * half;
            const size_t o = (size_t)gm * ld + gn;
            float d[4] = {d_of(g, 0) * rs, d_of(g, 1) * rs, d_of(g, 2) * rs, d_of(g, 3) * rs};
            if (vec_ok && gn + 3 < N) {
                if constexpr (OUT_F32) {
                    float4_t* const dst = reinterpret_cast<float4_t*>(static_cast<float*>(c) + o);
                    if (epi != kEpiStore) {
                        const float4_t old = *dst;
#pragma unroll
                        for (int r = 0; r < 4; ++r) d[r] = epilogue(epi, old[r], d[r]);
                    }
                    *dst = float4_t{d[0], d[1], d[2], d[3]};
                } else {
                    *reinterpret_cast<uint2_t*>(static_cast<uint16_t*>(c) + o) =
                        uint2_t{pack_bf16(d[0], d[1]), pack_bf16(d[2], d[3])};
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (gn + r < N) {
                        if constexpr (OUT_F32) {
                            float* const dst = static_cast<float*>(c) + o + r;
                            *dst = epi != kEpiStore ? epilogue(epi, *dst, d[r]) : d[r];
                        } else {
                            static_cast<uint16_t*>(c)[o + r] = (uint16_t)pack_bf16(d[r], 0.0f);
                        }
                    }
                }
            }
        }
    };
    if constexpr (FM % 2 == 0) {
        if (p.hilo) {
            // staged rows m0 + 64 i' .. + 63 are tokens m0 / 2 + 32 i' .. + 31: hi (tile 2 i'), lo (2 i' + 1)
#pragma unroll
            for (int i = 0; i < FM / 2; ++i) {
                const int gm = m0 / 2 + 32 * i + l32;
                if (gm >= p.m_out) continue;
                const float rs = p.splits > 1 ? 1.0f : p.row_scale[gm];
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    emit(gm, j, rs, [&](int g, int r) {
                        return acc[2 * i][j][4 * g + r] + acc[2 * i + 1][j][4 * g + r] * 0x1p-11f;
                    });
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int gm = m0 + 32 * i + l32;
        if (gm >= p.m_out) continue;
        const float rs = p.splits > 1 ? 1.0f : p.row_scale[gm];
#pragma unroll
        for (int j = 0; j < FN; ++j) emit(gm, j, rs, [&](int g, int r) { return acc[i][j][4 * g + r]; });
    }
}

// C[m][n] = row_scale[m] * sum_s partial[s][m][n], splits summed in order,
// written through the epilogue (fp32 C).  One thread per 4 consecutive
// outputs of a row.  Segment launches: columns [col[s], col[s] + n[s]) of the
// partial sums are segment s's output c[s] ([m][n[s]]; every n[s] a multiple
// of 4, so no 4-column group straddles two segments).
constexpr int kReduceThreads = 256;
constexpr int kMaxPrefillSplits = 16;  // plan_prefill splits K at most 16 ways

struct ReduceOut {
    int n_seg;  // 1: c[0] is [m][n]
    void* c[kMaxSegments];
    int n[kMaxSegments], col[kMaxSegments];
};

template <bool OUT_F32>
__global__ __launch_bounds__(kReduceThreads) void prefill_split_reduce(const float* __restrict__ partial,
                                                                       int splits, int m, int n,
                                                                       const float* __restrict__ row_scale,
                                                                       ReduceOut out, int epi) {
    const int n4 = (n + 3) >> 2;
    const size_t idx = (size_t)blockIdx.x * kReduceThreads + threadIdx.x;
    if (idx >= (size_t)m * n4) return;
    const int row = (int)(idx / n4);
    const int col = (int)(idx - (size_t)row * n4) * 4;
    const size_t stride = (size_t)m * n;
    const float rs = row_scale[row];
    const int cnt = min(4, n - col);
    float d[4] = {0.f, 0.f, 0.f, 0.f};
    int sg = 0;
    while (sg + 1 < out.n_seg && col >= out.col[sg + 1]) ++sg;
    void* const c = out.c[sg];
    const int nc = out.n_seg > 1 ? out.n[sg] : n;  // the output's row length
    const size_t oc = (size_t)row * nc + (col - (out.n_seg > 1 ? out.col[sg] : 0));
    const size_t o = (size_t)row * n + col;
    const bool vec = (n & 3) == 0 && (nc & 3) == 0 && ((uintptr_t)c & 15) == 0;
    if (vec) {
        // every split's load in flight before the first add (splits <= 16 is
        // uniform), then the sum in split order
        float4_t v[kMaxPrefillSplits];
#pragma unroll
        for (int sp = 0; sp < kMaxPrefillSplits; ++sp)
            if (sp < splits) v[sp] = *reinterpret_cast<const float4_t*>(partial + sp * stride + o);
#pragma unroll
        for (int sp = 0; sp < kMaxPrefillSplits; ++sp) {
            if (sp < splits) {
                d[0] += v[sp].x;
                d[1] += v[sp].y;
                d[2] += v[sp].z;
                d[3] += v[sp].w;
            }
        }
    } else {
        for (int sp = 0; sp < splits; ++sp)
            for (int r = 0; r < cnt; ++r) d[r] += partial[sp * stride + o + r];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) d[r] *= rs;
    if (vec) {
        if constexpr (OUT_F32) {
            float4_t* const dst = reinterpret_cast<float4_t*>(static_cast<float*>(c) + oc);
            if (epi != kEpiStore) {
                const float4_t old = *dst;
#pragma unroll
                for (int r = 0; r < 4; ++r) d[r] = epilogue(epi, old[r], d[r]);
            }
            *dst = float4_t{d[0], d[1], d[2], d[3]};
        } else {
            typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));
            *reinterpret_cast<uint2_t*>(static_cast<uint16_t*>(c) + oc) =
                uint2_t{pack_bf16(d[0], d[1]), pack_bf16(d[2], d[3])};
        }
    } else {
        for (int r = 0; r < cnt; ++r) {
            if constexpr (OUT_F32) {
                float* const dst = static_cast<float*>(c) + oc + r;
                *dst = epi != kEpiStore ? epilogue(epi, *dst, d[r]) : d[r];
            } else {
                static_cast<uint16_t*>(c)[oc + r] = (uint16_t)pack_bf16(d[r], 0.0f);
            }
        }
    }
}

template <int BM, int NW, int FN, int WPE, bool F16W = false, bool Q8W = false, int KH = 1, bool Q4W = false,
          bool SWI = false>
hipError_t launch_f16_tile(const PrefillArgs& a, bool out_f32, hipStream_t s) {
    constexpr int BN = (SWI && FN == 1 ? 16 : 32 * (SWI ? 1 : FN)) * NW / KH;
    const size_t lds = (size_t)token_buffers<BM>() * KH * BM * kLdsRow;
    if ((a.k_len / KH) % 256 != 0) return hipErrorInvalidValue;  // whole four-step loop bodies per half
    PrefillArgs p = a;
    p.tiles_m = (a.m + BM - 1) / BM;
    p.tiles_n = (a.n + BN - 1) / BN;
    if (a.n_seg > 1) {
        p.tiles_n = 0;
        for (int s = 0; s < a.n_seg; ++s) {
            p.seg_tiles[s] = (a.seg_n[s] + BN - 1) / BN;
            p.tiles_n += p.seg_tiles[s];
        }
    }
    const dim3 grid(p.tiles_m * p.tiles_n * p.splits);
    if (a.info) {
        // every template argument, as the profiler names the instantiation
        snprintf(a.info->name, sizeof a.info->name, "gf4_prefill_f16_kernel<%d, %d, %d, %d, %s, %s, %s, %d, %s, %s>",
                 BM, NW, FN, WPE, out_f32 ? "true" : "false", F16W ? "true" : "false", Q8W ? "true" : "false", KH,
                 Q4W ? "true" : "false", SWI ? "true" : "false");
        a.info->grid = grid.x;
        a.info->block = 64u * NW;
        a.info->lds = (unsigned)lds;
        a.info->splits = (unsigned)p.splits;
        return hipSuccess;
    }
    if constexpr (SWI) {
        if (!out_f32) return hipErrorInvalidValue;
        hipLaunchKernelGGL((gf4_prefill_f16_kernel<BM, NW, FN, WPE, true, false, false, KH, false, true>), grid,
                           dim3(64 * NW), lds, s, p);
    } else if (out_f32) {
        hipLaunchKernelGGL((gf4_prefill_f16_kernel<BM, NW, FN, WPE, true, F16W, Q8W, KH, Q4W>), grid, dim3(64 * NW), lds,
                           s, p);
    } else {
        hipLaunchKernelGGL((gf4_prefill_f16_kernel<BM, NW, FN, WPE, false, F16W, Q8W, KH, Q4W>), grid, dim3(64 * NW), lds,
                           s, p);
    }
    return hipGetLastError();
}

template <int BM, int BN, int WGM, int WGN>
hipError_t launch_tile(const PrefillArgs& a, bool a_f32, bool has_awq, bool out_f32, hipStream_t s) {
    constexpr int NT = 64 * WGM * WGN;
    const size_t lds = 2 * (size_t)(BM + BN) * kLdsRow;
    PrefillArgs p = a;
    p.tiles_m = (a.m + BM - 1) / BM;
    p.tiles_n = (a.n + BN - 1) / BN;
    const dim3 grid(p.tiles_m * p.tiles_n);
    if (a.info) {
        snprintf(a.info->name, sizeof a.info->name, "gf4_prefill_kernel<%d, %d, %d, %d, %s, %s, %s>", BM, BN, WGM, WGN,
                 a_f32 ? "true" : "false", has_awq ? "true" : "false", out_f32 ? "true" : "false");
        a.info->grid = grid.x;
        a.info->block = (unsigned)NT;
        a.info->lds = (unsigned)lds;
        a.info->splits = 1;
        return hipSuccess;
    }
#define QW35_PF(AF, AW, OF) \
    hipLaunchKernelGGL((gf4_prefill_kernel<BM, BN, WGM, WGN, AF, AW, OF>), grid, dim3(NT), lds, s, p)
    if (a_f32) {
        if (has_awq) {
            if (out_f32) QW35_PF(true, true, true); else QW35_PF(true, true, false);
        } else {
            if (out_f32) QW35_PF(true, false, true); else QW35_PF(true, false, false);
        }
    } else {
        if (has_awq) {
            if (out_f32) QW35_PF(false, true, true); else QW35_PF(false, true, false);
        } else {
            if (out_f32) QW35_PF(false, false, true); else QW35_PF(false, false, false);
        }
    }
#undef QW35_PF
    return hipGetLastError();
}

// MFMA throughput probe: each wave runs `iters` rounds of 8 independent
// v_mfma_f32_32x32x16_f16 (the prefill kernel's instruction) with no memory
// traffic; one float per thread goes to sink so the work stays live.
constexpr int kProbeThreads = 256;

__global__ __launch_bounds__(kProbeThreads) void mfma_probe_kernel(int iters, float* __restrict__ sink) {
    typedef float float16_t __attribute__((ext_vector_type(16)));
    half8_t a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (_Float16)((float)((threadIdx.x + i) & 15) * 0x1p-12f);
        b[i] = (_Float16)((float)(i + 1) * 0x1p-10f);
    }
    float16_t acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[j][r];
    sink[(size_t)blockIdx.x * kProbeThreads + threadIdx.x] = s;
}

int num_cus() {
    static int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            return 256;
        }
        return n;
    }();
    return cus;
}

size_t round256(size_t b) { return (b + 255) / 256 * 256; }

}  // namespace

// Staged-path launch shape from a cost model fitted to MI355X measurements of
// the Qwen3.5-9B projection shapes (M = 128..2048): the grid runs in
// ceil(blocks / CUs) rounds; a block costs 0.108 us per MFLOP of MFMA work
// plus 29.9 us per MB it streams (its token tile once per k step, its weight
// slab once); a K split adds 0.5 us per MB of fp32 partial sums (written,
// read back by the reduction, one more launch).  Over the measured shapes the
// pick is the fastest or within 5% of it.
// F16 weights (2 bytes per weight against GF4's half byte) use FN = 2 only:
// their four-slot register ring of 16-byte loads is four times GF4's.
// fp32 input (hilo) stages two rows per token in 32-token groups: the tiles
// are planned over the staged rows, of at least 64 (one hi and one lo MFMA
// tile per wave), and the K-split partial sums stay one row per token.
// Q4_K blocks (q4w) plan as q8_0 blocks do (the same load ring and one-tile
// waves), with their own bytes per weight.
PrefillCfg plan_prefill(int m_tokens, int rows, int k, bool f16w, bool q8w, bool hilo, bool q4w = false) {
    const int m = staged_rows(m_tokens, hilo);
    const double w_bytes = f16w ? 2.0 : q4w ? 144.0 / 256.0 : q8w ? 34.0 / 32.0 : 0.5;
    q8w = q8w || q4w;
    constexpr double kUsPerMflop = 0.108, kUsPerMB = 29.9;
    // K-split partial sums cost less relative to fp16 weight tiles than to GF4
    // ones: with 0.5 the F16 plan for 8192x4096 M=128 was {64,2,4} 57.1 us,
    // with 0.35 it is {128,2,8} 47.0 us; the other F16 shapes of the sweep
    // (4096 / 8192 / 12288 rows, M = 128..2048) keep their plans.
    // q8_0 in-kernel (sweep on 8192x4096 M = 512): split 2 of 128-token tiles
    // 100 us, 64-token tiles unsplit 140 us; with 0.5 the model picked the latter.
    const double kUsPerPartialMB = (f16w || q8w) ? 0.35 : 0.5;
    const int cus = num_cus();
    const int chunks = k / 256;
    // 256-token tiles (one wave per SIMD, 256 accumulator registers) only for
    // F16 and q8_0 weights: q8_0 8192x4096 M = 2048 200 us against 331 with
    // 128 tokens, F16 172 against 244; GF4 was slower with them (236-260 us
    // against 210 at 12288x4096).
    static constexpr int kShapes[][2] = {{256, 2}, {128, 4}, {128, 2}, {64, 4}, {64, 2}, {32, 2}};
    PrefillCfg best{hilo ? 64 : 32, 2, 1};
    double best_us = 0;
    for (const auto& sh : kShapes) {
        const int bm = sh[0], fn = sh[1], bn = 128 * fn;
        if ((f16w || q8w) && fn != 2) continue;
        if (bm == 256 && !(f16w || q8w)) continue;
        if (bm == 256 && q4w) continue;  // its 8-wave 256-token tile spills registers
        if (bm > 32 && m <= bm / 2) continue;  // half the token tile or more would be padding
        if (hilo && bm < 64) continue;
        const long tiles = (long)((m + bm - 1) / bm) * ((rows + bn - 1) / bn);
        for (int sp = 1; sp <= 16 && sp <= chunks; ++sp) {
            if (chunks % sp != 0 || (sp > 1 && k / sp < 512)) continue;
            const long blocks = tiles * sp;
            const double rounds = (double)((blocks + cus - 1) / cus);
            const double k_len = (double)k / sp;
            double us = rounds * (kUsPerMflop * 2.0 * bm * bn * k_len * 1e-6 + kUsPerMB * k_len * (2.0 * bm + w_bytes * bn) * 1e-6);
            if (sp > 1) us += kUsPerPartialMB * 4.0 * sp * m_tokens * rows * 1e-6;
            if (best_us == 0 || us < best_us) {
                best_us = us;
                best = {bm, fn, sp};
            }
            if (blocks >= cus) break;  // more splits only add partial sums
        }
    }
    // One block per CU or fewer: the 8-wave form of the same tile hides more
    // latency.  Same-box A/B, GF4: 12288x4096 M=128 {64,2,2} 37.7 -> 35.8 us,
    // M=512 {128,2,1} 76.4 -> 71.2 us; 4096x12288 M=512 {128,2,4} 75.7 ->
    // 72.9 us.  At three blocks per CU (M=2048) it was slower, 216 -> 233 us.
    const long blocks = (long)((m + best.bm - 1) / best.bm) * ((rows + 255) / 256) * best.splits;
    if (!f16w && best.fn == 2 && best.bm >= 64 && blocks <= cus) best.waves = 8;
    // q8_0: three 16-byte loads per 32-row tile and step in a four-slot ring
    // (96 VGPRs at two tiles per wave), so a 256-row tile of 64 or more
    // tokens always runs on 8 waves of one tile each.
    if (q8w && best.bm >= 64 && best.bm <= 128) best.waves = 8;
    // 256-token tiles (F16 and q8_0 weights): 8 one-tile waves, two per SIMD
    // (128 accumulator registers each) in place of 4 two-tile waves.  Sweep
    // after the cached weight loads (us, 4 -> 8 waves): F16 12352x4096 M =
    // 1024 / 2048 147.7 -> 131.9 / 275.4 -> 243.2, 8192x4096 M = 2048 149.6 ->
    // 140.1; q8_0 12352x4096 M = 2048 275.9 -> 261.6, 8192x4096 156.4 -> 148.8.
    if ((f16w || q8w) && best.bm == 256) best.waves = 8;
    // A 256-row tile on 8 one-tile waves with an even K split does the same
    // work as a 128-row tile whose two K halves run on four waves each and are
    // summed in LDS, with half the splits: half the fp32 partial sums, and no
    // reduction launch where the split was two, for twice the token-tile
    // reads.  Same-box A/B (us, without -> with): GF4 12288x4096 M = 128
    // 35.0 -> 31.9, 4096x12288 M = 128 37.1 -> 35.5; q8_0 8192x4096 M = 128 /
    // 512 57.3 -> 54.3 / 95.1 -> 83.4, 4096x4096 38.2 -> 35.1 / 60.1 -> 55.4.
    // GF4 tiles of 128 tokens keep a split of more than two (4096x12288
    // M = 512: 69.4 -> 74.0 with the halves).
    if (!f16w && best.waves == 8 && best.fn == 2 && best.bm <= 128 && best.splits % 2 == 0 &&
        (q8w || best.bm <= 64 || best.splits == 2)) {
        best.kh = 2;
        best.splits /= 2;
    }
    // q8_0 over one token tile of at most 64 staged rows: K parts of down to
    // 256 columns (the K halves of 512-column splits) until the grid fills the
    // CUs once; the cost model stops at 512-column splits.  Same box, µs,
    // plan -> more splits: 4096x4096 fp32 9 / 32 tokens 21.3 / 21.9 -> 16.8 /
    // 18.4, bf16 16 / 64 tokens 20.5 / 22.7 -> 16.4 / 21.0; 2048x4096 fp32 9
    // tokens 20.7 -> 15.4 (grids of more row tiles keep their plans).
    if (q8w && !q4w && m <= 64 && best.bm == 64 && best.waves == 8 && best.kh == 2) {
        const long tiles = (rows + 127) / 128;
        while (tiles * best.splits * 2 <= cus && best.splits * 2 <= 16 && k % (best.splits * 2 * 2 * 256) == 0)
            best.splits *= 2;
    }
    // Q4_K: every block dequantises its whole weight tile on the VALU, so a
    // 64-token tile over more than 64 tokens decodes each weight twice as
    // often as a 128-token tile; take the latter with twice the K split.
    // Same-box sweep, bf16 activations, 4096x12288 M = 128: {64, split 4,
    // halves} 44.0 us -> {128, split 8, halves} 37.3 us.
    if (q4w && !hilo && best.bm == 64 && m > 64 && 2 * best.splits <= 16 && chunks % (2 * best.splits * best.kh) == 0 &&
        k / (2 * best.splits * best.kh) >= 512) {
        best.bm = 128;
        best.splits *= 2;
    }
    // K quarters for GF4 at 33..128 tokens and k <= 4096: each 64-token block
    // runs four parts of its K range (16 steps each at k = 4096, summed in
    // LDS) instead of two of 32, with no K split and so no reduction launch,
    // on 8 waves over 64 rows, 12 over 96 or 16 over 128, the first that
    // fills half the CUs to all of them in one round.
    // Same-box A/B at M = 128 (us, plan -> quarters): 8192x4096 28.3 -> 22.0
    // (8 waves), 4096x4096 21.5 -> 19.9 (8), 12288x4096 29.5 -> 28.0 (16
    // waves); 4096x12288 (48-step quarters) was not faster, 30.5 -> 30.5-36.4.
    // 12 waves (three per SIMD) give 12288 rows of two token tiles 256 blocks
    // in place of 192 of 16 waves: same box, 16 -> 12 waves, us: bf16 M = 128
    // 29.5-31.4 -> 28.1, M = 96 28.1-28.4 -> 26.7; fp32 M = 64 28.8-29.5 ->
    // 27.7-28.2, M = 48 28.3-28.6 -> 26.7-27.0.
    if (!f16w && !q8w && m > 32 && m <= 128 && k <= 4096 && k % 1024 == 0) {
        const long tm = (m + 63) / 64;
        const long b64 = tm * ((rows + 63) / 64), b96 = tm * ((rows + 95) / 96), b128 = tm * ((rows + 127) / 128);
        const int waves = 2 * b64 >= cus && b64 <= cus     ? 8
                          : 2 * b96 >= cus && b96 <= cus   ? 12
                          : 2 * b128 >= cus && b128 <= cus ? 16
                                                           : 0;
        if (waves) {
            best.bm = 64;
            best.fn = 2;
            best.splits = 1;
            best.waves = waves;
            best.kh = 4;
        }
    }
    // fp32 activations of 65..128 tokens (129..256 staged rows) on GF4 rows of
    // k <= 4096: a 128-row tile on 8 waves as two K halves, unsplit (same box,
    // 12288x4096 M = 128: 47.0-50.5 us planned {128, fn 4, 4 splits} -> 40.3;
    // 4096x12288 kept its plan, 41.1 against 42.3-149 us for the others).
    if (hilo && !f16w && !q8w && m > 128 && m <= 256 && k <= 4096 && k % 512 == 0) {
        best = PrefillCfg{128, 2, 1};
        best.waves = 8;
        best.kh = 2;
    }
    return best;
}

PrefillCfg plan_prefill_kind(int m, int rows, int k, int wkind, bool a_f32) {
    return plan_prefill(m, rows, k, wkind == 1, wkind == 2, a_f32, wkind == 3);
}

PrefillCfg plan_gf4_prefill(int m, int rows, int k, bool a_f32) { return plan_prefill_kind(m, rows, k, 0, a_f32); }

// Staged tokens (2 bytes per staged activation), one fp32 scale per token,
// then the K-split partial sums (fp32, one row per token and split).
size_t gf4_prefill_workspace_bytes(int m, int rows, int k, PrefillCfg cfg, bool a_f32) {
    size_t b = round256((size_t)staged_rows(m, a_f32) * k * 2) + round256((size_t)m * 4);
    if (cfg.splits > 1) b += (size_t)cfg.splits * m * rows * 4;
    return b;
}

size_t prefill_workspace_bytes(int m, int rows, int k, int wkind, bool with_f32) {
    const size_t b16 = gf4_prefill_workspace_bytes(m, rows, k, plan_prefill_kind(m, rows, k, wkind, false), false);
    if (!with_f32) return b16;
    const size_t b32 = gf4_prefill_workspace_bytes(m, rows, k, plan_prefill_kind(m, rows, k, wkind, true), true);
    return b16 > b32 ? b16 : b32;
}

size_t prefill_min_workspace_bytes(int m, int rows, int k, bool a_f32) {
    return gf4_prefill_workspace_bytes(m, rows, k, PrefillCfg{64, 2, 1}, a_f32);
}

namespace {

// A workspace sized for another token count may not hold this call's partial
// sums: split less (ultimately not at all) rather than fail; K halves need
// each half to stay a multiple of 256 columns.
void fit_prefill_workspace(int m, int rows, int k, PrefillCfg& cfg, size_t workspace_bytes, bool a_f32) {
    while (cfg.splits > 1 && gf4_prefill_workspace_bytes(m, rows, k, cfg, a_f32) > workspace_bytes) {
        do --cfg.splits;
        while (cfg.splits > 1 && (k % cfg.splits != 0 || (k / cfg.splits) % (256 * cfg.kh) != 0));
    }
    if ((k / cfg.splits) % (256 * cfg.kh) != 0) cfg.kh = 1;
}

// The gate launches the fused gate/up kernel replaces: GF4 words, unsplit, 8
// waves of one 32-row weight tile each over 64 or 128 tokens, with K halves,
// quarters (64 tokens) or neither; the fused kernel then holds a gate and an
// up tile per wave.  q8_0 and Q4_K hold three 16-byte loads per tile in their
// load ring.  The 16-wave quarters would spill; a fused 12-wave form ran about
// the same (same box, 12288x4096: 43-44 us against 44-45 for the 8-wave K
// halves at 48-64 tokens, 79 against 68-70 at 128 tokens) and is not built.
bool swiglu_tile_ok(int wkind, const PrefillCfg& cfg) {
    if (wkind != 0 || cfg.splits != 1 || cfg.fn != 2 || cfg.waves != 8) return false;
    if (cfg.kh == 4) return cfg.bm == 64;
    return (cfg.kh == 1 || cfg.kh == 2) && (cfg.bm == 64 || cfg.bm == 128);
}

// A fused launch's configuration: those tiles, or their mixed form (12 waves;
// the 12-wave K quarters of an unfused plan are not one).
bool swiglu_cfg_ok(int wkind, const PrefillCfg& cfg) {
    if (wkind != 0 || cfg.splits != 1 || cfg.fn != 2) return false;
    if (cfg.waves == 12)
        return (cfg.bm == 128 && (cfg.kh == 1 || cfg.kh == 2)) || (cfg.bm == 64 && (cfg.kh == 2 || cfg.kh == 4));
    return swiglu_tile_ok(wkind, cfg);
}

// The fused gate/up launch of m tokens (fp32 input: the runtime's chunks):
// the gate's own plan where it has the fused form; else, for fp32 input,
//  * in place of the 12- or 16-wave 64-token K quarters (33..64 tokens): the
//    8-wave 64-token tile with K halves;
//  * in place of a split plan at 129..256 tokens: the unsplit 8-wave
//    128-token tile,
// where the fused grid still gives at least half the CUs a block.  Same box,
// GF4 12288x4096, gate/up as one op, us (two launches -> fused): 48 tokens
// 55.0 -> 44.5, 64 tokens 56.2 -> 45.3, 192 tokens 138.5 -> 95.3, 256 tokens
// 147.9 -> 105.5.  The gate's own plan gives the two launches' bits; the
// others sum K in another grouping (within fp32 rounding of them).  False:
// the op runs as the gate and up launches.
bool plan_swiglu(int wkind, int m, int rows, int k, bool a_f32, size_t workspace_bytes, PrefillCfg& cfg) {
    cfg = plan_prefill_kind(m, rows, k, wkind, a_f32);
    fit_prefill_workspace(m, rows, k, cfg, workspace_bytes, a_f32);
    // An 8-wave fused tile as mixed tiles (three waves per SIMD, 16 rows per
    // wave of a K part: 192 rows per block without K parts, 96 with K halves,
    // 48 with quarters) where that grid fills more CUs in one round; the same
    // K partition, so the same bits.
    auto mixed = [&](PrefillCfg& c) {
        if (c.waves != 8 || c.splits != 1 || (c.kh == 4 && c.bm != 64) || (c.kh == 1 && c.bm != 128)) return;
        const long tm = (staged_rows(m, a_f32) + c.bm - 1) / c.bm;
        const int rows_mixed = 192 / c.kh, rows_two = 256 / c.kh;
        // without K parts only up to three token tiles: at four (193..256
        // tokens) the mixed form was 0.5-1% slower (same box, gate/up op at
        // 224 / 256 tokens 103.7 / 105.8 -> 104.2 / 106.7 us; 129 / 192
        // tokens 87.7 / 90.7 -> 80.1 / 88.3)
        if (c.kh == 1 && tm > 3) return;
        const long b_mixed = tm * ((rows + rows_mixed - 1) / rows_mixed), b_two = tm * ((rows + rows_two - 1) / rows_two);
        if (b_mixed > b_two && b_mixed <= num_cus()) c.waves = 12;
    };
    if (swiglu_tile_ok(wkind, cfg)) {
        mixed(cfg);
        return true;
    }
    if (wkind != 0 || !a_f32) return false;
    const int ms = staged_rows(m, a_f32);
    PrefillCfg alt{64, 2, 1};
    alt.waves = 8;
    long blocks = 0;
    if (cfg.bm == 64 && cfg.kh == 4 && cfg.waves > 8 && k % 512 == 0) {
        alt.kh = 2;  // 64 tokens by 128 rows per block
        blocks = (long)((ms + 63) / 64) * ((rows + 127) / 128);
    } else if (ms > 256 && ms <= 512) {
        alt.bm = 128;  // 128 tokens by 256 rows per block
        blocks = (long)((ms + 127) / 128) * ((rows + 255) / 256);
    }
    if (2 * blocks < num_cus()) return false;
    cfg = alt;
    mixed(cfg);
    return true;
}

}  // namespace

// wkind: 0 GF4 words, 1 F16 weights, 2 q8_0 blocks, 3 Q4_K super-blocks (1..3 take column-order tokens and a
// workspace).
hipError_t launch_gf4_prefill_cfg(const void* w, int rows, int k, const void* a, int a_f32, const float* awq,
                                  void* c, int m, int out_f32, void* workspace, PrefillCfg cfg,
                                  hipStream_t stream, int wkind, int epi, LaunchInfo* info, bool staged,
                                  const PrefillSegs* segs, const void* w_up) {
    const bool f16w = wkind == 1, q8w = wkind == 2, q4w = wkind == 3;
    PrefillArgs p{};
    p.w = static_cast<const uint32_t*>(w);
    p.w_up = static_cast<const uint32_t*>(w_up);
    // fused gate/up: the configurations prefill_swiglu_fusable accepts, STORE of silu(g) * u
    if (w_up && (!swiglu_cfg_ok(wkind, cfg) || !workspace || !out_f32 || epi != kEpiStore || (segs && segs->n > 1)))
        return hipErrorInvalidValue;
    p.a = a;
    p.awq = awq;
    p.c = c;
    p.m = m;
    p.m_out = m;
    p.hilo = 0;
    p.epi = epi;
    p.info = info;
    // epilogues read fp32 c; the path without a workspace has none
    if (epi != kEpiStore && (!out_f32 || !workspace)) return hipErrorInvalidValue;
    if (epi < kEpiStore || epi > kEpiSwiglu) return hipErrorInvalidValue;
    ReduceOut out{};
    out.n_seg = 1;
    out.c[0] = c;
    if (segs && segs->n > 1) {
        // segments: staged path only, rows = their sum, each a multiple of 4
        if (!workspace || segs->n > kMaxSegments) return hipErrorInvalidValue;
        int total = 0;
        for (int s = 0; s < segs->n; ++s) {
            if (segs->rows[s] < 1 || segs->rows[s] % 4 != 0 || !segs->w[s] || !segs->c[s])
                return hipErrorInvalidValue;
            p.seg_w[s] = segs->w[s];
            p.seg_c[s] = segs->c[s];
            p.seg_n[s] = segs->rows[s];
            p.seg_col[s] = total;
            out.c[s] = segs->c[s];
            out.n[s] = segs->rows[s];
            out.col[s] = total;
            total += segs->rows[s];
        }
        if (total != rows) return hipErrorInvalidValue;
        p.n_seg = out.n_seg = segs->n;
    }
    p.n = rows;
    p.k = k;
    p.splits = 1;
    p.k_len = k;
    bool af = a_f32 != 0, aw = awq != nullptr;
    const bool of = out_f32 != 0;
    if (workspace) {
        if (cfg.splits < 1 || cfg.splits > kMaxPrefillSplits || (cfg.kh != 1 && cfg.kh != 2 && cfg.kh != 4) ||
            k % cfg.splits != 0 ||
            (k / cfg.splits) % (256 * cfg.kh) != 0)
            return hipErrorInvalidValue;
        // fp32 input: hi and lo tiles pair up inside a wave's token tiles
        if (af && cfg.bm < 64) return hipErrorInvalidValue;
        // K halves exist for the 8-wave 64- and 128-token tiles of GF4 and q8_0 weights only
        if (cfg.kh == 2 && (f16w || (cfg.waves != 8 && !(w_up && cfg.waves == 12)) || cfg.fn != 2 ||
                            (cfg.bm != 64 && cfg.bm != 128)))
            return hipErrorInvalidValue;
        // K quarters: the 64-token GF4 tile on 16 waves (128 rows), 12 (96) or 8 (64)
        if (cfg.kh == 4 &&
            (f16w || q8w || q4w || (cfg.waves != 16 && cfg.waves != 12 && cfg.waves != 8) || cfg.fn != 2 || cfg.bm != 64))
            return hipErrorInvalidValue;
        const int ms = staged_rows(m, af);
        uint8_t* ws = static_cast<uint8_t*>(workspace);
        uint16_t* a16 = reinterpret_cast<uint16_t*>(ws);
        float* rs = reinterpret_cast<float*>(ws + round256((size_t)ms * k * 2));
        float* partial = reinterpret_cast<float*>(ws + round256((size_t)ms * k * 2) + round256((size_t)m * 4));
        const unsigned stage_grid = af ? (unsigned)(ms / 2) : (unsigned)m;
        if (info) info->ws_bytes = gf4_prefill_workspace_bytes(m, rows, k, cfg, af);
#define QW35_STAGE(AF, AW, ORD) launch_stage<AF, AW, ORD>(stage_grid, stream, a, awq, m, k, a16, rs)
        if (info || staged) {
            // described only, or the workspace already holds these activations staged
        } else if (f16w || q8w || q4w) {
            if (af) {
                if (aw) QW35_STAGE(true, true, false); else QW35_STAGE(true, false, false);
            } else {
                if (aw) QW35_STAGE(false, true, false); else QW35_STAGE(false, false, false);
            }
        } else {
            if (af) {
                if (aw) QW35_STAGE(true, true, true); else QW35_STAGE(true, false, true);
            } else {
                if (aw) QW35_STAGE(false, true, true); else QW35_STAGE(false, false, true);
            }
        }
#undef QW35_STAGE
        hipError_t e = info || staged ? hipSuccess : hipGetLastError();
        if (e != hipSuccess) return e;
        p.a = a16;
        p.awq = nullptr;
        p.row_scale = rs;
        p.m = ms;
        p.hilo = af ? 1 : 0;
        p.splits = cfg.splits;
        p.k_len = k / cfg.splits;
        const bool split = cfg.splits > 1;
        if (split) p.c = partial;
        const bool kf32 = of || split;
        if (w_up) {
            if (cfg.waves == 12) {  // mixed tiles: three waves per SIMD
                if (cfg.bm == 128)
                    return cfg.kh == 1 ? launch_f16_tile<128, 12, 1, 3, false, false, 1, false, true>(p, true, stream)
                                       : launch_f16_tile<128, 12, 1, 3, false, false, 2, false, true>(p, true, stream);
                return cfg.kh == 4 ? launch_f16_tile<64, 12, 1, 3, false, false, 4, false, true>(p, true, stream)
                                   : launch_f16_tile<64, 12, 1, 3, false, false, 2, false, true>(p, true, stream);
            }
            if (cfg.bm == 128)
                return cfg.kh == 2 ? launch_f16_tile<128, 8, 2, 2, false, false, 2, false, true>(p, true, stream)
                                   : launch_f16_tile<128, 8, 2, 2, false, false, 1, false, true>(p, true, stream);
            // K quarters: two waves per SIMD (a gate and an up tile per wave
            // need more than the 128 VGPRs of the unfused form's four)
            if (cfg.kh == 4) return launch_f16_tile<64, 8, 2, 2, false, false, 4, false, true>(p, true, stream);
            return cfg.kh == 2 ? launch_f16_tile<64, 8, 2, 2, false, false, 2, false, true>(p, true, stream)
                               : launch_f16_tile<64, 8, 2, 2, false, false, 1, false, true>(p, true, stream);
        }
        if (q4w) {  // no 256-token tiles (plan_prefill never picks them for Q4_K)
            switch (cfg.bm * 10 + cfg.fn) {
                case 1282:
                    e = cfg.kh == 2 ? launch_f16_tile<128, 8, 1, 2, false, false, 2, true>(p, kf32, stream)
                                    : launch_f16_tile<128, 8, 1, 2, false, false, 1, true>(p, kf32, stream);
                    break;
                case 642:
                    e = cfg.kh == 2 ? launch_f16_tile<64, 8, 1, 2, false, false, 2, true>(p, kf32, stream)
                                    : launch_f16_tile<64, 8, 1, 2, false, false, 1, true>(p, kf32, stream);
                    break;
                case 322: e = launch_f16_tile<32, 4, 2, 2, false, false, 1, true>(p, kf32, stream); break;
                default: return hipErrorInvalidValue;
            }
        } else if (q8w) {
            switch (cfg.bm * 10 + cfg.fn) {
                case 2562:
                    e = cfg.waves == 8 ? launch_f16_tile<256, 8, 1, 2, false, true>(p, kf32, stream)
                                       : launch_f16_tile<256, 4, 2, 1, false, true>(p, kf32, stream);
                    break;
                case 1282:
                    e = cfg.kh == 2 ? launch_f16_tile<128, 8, 1, 2, false, true, 2>(p, kf32, stream)
                                    : launch_f16_tile<128, 8, 1, 2, false, true>(p, kf32, stream);
                    break;
                case 642:
                    e = cfg.kh == 2 ? launch_f16_tile<64, 8, 1, 2, false, true, 2>(p, kf32, stream)
                                    : launch_f16_tile<64, 8, 1, 2, false, true>(p, kf32, stream);
                    break;
                case 322: e = launch_f16_tile<32, 4, 2, 2, false, true>(p, kf32, stream); break;
                default: return hipErrorInvalidValue;
            }
        } else if (f16w) {
            switch (cfg.bm * 10 + cfg.fn) {
                case 2562:
                    e = cfg.waves == 8 ? launch_f16_tile<256, 8, 1, 2, true>(p, kf32, stream)
                                       : launch_f16_tile<256, 4, 2, 1, true>(p, kf32, stream);
                    break;
                case 1282: e = launch_f16_tile<128, 4, 2, 1, true>(p, kf32, stream); break;
                case 642: e = launch_f16_tile<64, 4, 2, 2, true>(p, kf32, stream); break;
                case 322: e = launch_f16_tile<32, 4, 2, 2, true>(p, kf32, stream); break;
                default: return hipErrorInvalidValue;
            }
        } else switch (cfg.bm * 10 + cfg.fn) {
            case 1282:
                e = cfg.kh == 2      ? launch_f16_tile<128, 8, 1, 2, false, false, 2>(p, kf32, stream)
                    : cfg.waves == 8 ? launch_f16_tile<128, 8, 1, 2>(p, kf32, stream)
                                     : launch_f16_tile<128, 4, 2, 2>(p, kf32, stream);
                break;
            case 1284: e = launch_f16_tile<128, 4, 4, 1>(p, kf32, stream); break;
            case 642:
                e = cfg.kh == 4      ? (cfg.waves == 16   ? launch_f16_tile<64, 16, 1, 4, false, false, 4>(p, kf32, stream)
                                        : cfg.waves == 12 ? launch_f16_tile<64, 12, 1, 4, false, false, 4>(p, kf32, stream)
                                                          : launch_f16_tile<64, 8, 1, 4, false, false, 4>(p, kf32, stream))
                    : cfg.kh == 2    ? launch_f16_tile<64, 8, 1, 2, false, false, 2>(p, kf32, stream)
                    : cfg.waves == 8 ? launch_f16_tile<64, 8, 1, 2>(p, kf32, stream)
                                     : launch_f16_tile<64, 4, 2, 2>(p, kf32, stream);
                break;
            case 644: e = launch_f16_tile<64, 4, 4, 2>(p, kf32, stream); break;
            case 322: e = launch_f16_tile<32, 4, 2, 2>(p, kf32, stream); break;
            default: return hipErrorInvalidValue;
        }
        if (e != hipSuccess || !split || info) return e;
        const size_t threads = (size_t)m * ((rows + 3) / 4);
        const dim3 grid((unsigned)((threads + kReduceThreads - 1) / kReduceThreads));
        if (of)
            hipLaunchKernelGGL((prefill_split_reduce<true>), grid, dim3(kReduceThreads), 0, stream, partial,
                               cfg.splits, m, rows, rs, out, epi);
        else
            hipLaunchKernelGGL((prefill_split_reduce<false>), grid, dim3(kReduceThreads), 0, stream, partial,
                               cfg.splits, m, rows, rs, out, kEpiStore);
        return hipGetLastError();
    }
    // Direct path: largest tile that still gives every CU a block.
    if (p.n_seg > 1) return hipErrorInvalidValue;
    const long cus = num_cus();
    auto tiles = [&](int bm, int bn) { return (long)((m + bm - 1) / bm) * ((rows + bn - 1) / bn); };
    if (!af && tiles(256, 128) >= cus) return launch_tile<256, 128, 4, 2>(p, af, aw, of, stream);
    if (tiles(128, 128) >= cus) return launch_tile<128, 128, 2, 2>(p, af, aw, of, stream);
    return launch_tile<64, 64, 2, 2>(p, af, aw, of, stream);
}

hipError_t launch_prefill(int wkind, const void* w, int rows, int k, const void* a, int a_f32, const float* awq,
                          void* c, int m, int out_f32, void* workspace, size_t workspace_bytes, hipStream_t stream,
                          int epi, LaunchInfo* info, bool staged, const PrefillSegs* segs, const void* w_up) {
    if (!workspace && wkind != 0) return hipErrorInvalidValue;
    if (staged && !workspace) return hipErrorInvalidValue;
    PrefillCfg cfg = plan_prefill_kind(m, rows, k, wkind, a_f32 != 0);
    if (workspace) fit_prefill_workspace(m, rows, k, cfg, workspace_bytes, a_f32 != 0);
    if (w_up && !plan_swiglu(wkind, m, rows, k, a_f32 != 0, workspace_bytes, cfg)) return hipErrorInvalidValue;
    return launch_gf4_prefill_cfg(w, rows, k, a, a_f32, awq, c, m, out_f32, workspace, cfg, stream, wkind, epi, info,
                                  staged, segs, w_up);
}

bool prefill_swiglu_fusable(int wkind, int m, int rows, int k, int a_f32, size_t workspace_bytes) {
    PrefillCfg cfg{};
    return plan_swiglu(wkind, m, rows, k, a_f32 != 0, workspace_bytes, cfg);
}

hipError_t launch_mfma_probe(unsigned workgroups, unsigned iters, float* sink, hipStream_t stream) {
    hipLaunchKernelGGL(mfma_probe_kernel, dim3(workgroups), dim3(kProbeThreads), 0, stream, (int)iters, sink);
    return hipGetLastError();
}


}  // namespace qw35
