// GF4 prefill dequant-matmul on bf16 MFMA (gfx950):
//
//   C[m][n] = sum_k bf16_rne(awq[k] * A[m][k]) * W[n][k]        (awq == nullptr: A[m][k])
//
// A: [M][K] bf16 (or fp32) activations, W: GF4 tensor [N][K], C: [M][N] bf16 (RNE)
// or fp32, fp32 accumulation.  This is the tiled multi-token matmul of
// encodeMatvecBatch / encodeTiledKMatmul for type 100
// (qw35-server/src/metal/bridge/Qw35MetalRuntime+FFN.m:260-366, kernel
// qw35_mul_mm_gf4_f32 in qw35_tiled_mm.metal:203-255), designed for CDNA4:
//
// * A block computes a BM x BN tile of C with WGM x WGN waves; each wave owns a
//   (BM/WGM) x (BN/WGN) sub-tile of 16x16 v_mfma_f32_16x16x32_bf16 accumulators.
// * Per 64-wide k step the block stages A and the dequantised W tile as bf16 in
//   LDS (double buffered, 16-byte row padding against bank conflicts).  The next
//   step's global loads are issued before the MFMAs of the current one, and
//   their conversion (AWQ multiply + RNE for A, GF4 decode for W) follows them.
// * GF4 decode is exact in bf16: w_i = -sext3(c_i) * s / 4, s = fp16(b << 8)
//   (the format of tools/qw35_cook_common.py:79 with c = q_raw ^ 4).
// * Blocks are assigned XCD by XCD (consecutive block ids land on different
//   XCDs), M-tile fastest, so the blocks that share a W tile share an L2.
#include "qw35_device.h"
#include "qw35_kernels.h"

namespace qw35 {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

constexpr int kBK = 64;                 // k per pipeline step: 8 GF4 words per W row
constexpr int kLdsRow = kBK * 2 + 16;   // bytes per staged row: 64 bf16 + 16 B pad
constexpr int kXcds = 8;

struct PrefillArgs {
    const uint32_t* w;   // GF4 words [N][K/8]
    const void* a;       // [M][K] bf16 or fp32
    const float* awq;    // [K] or nullptr
    void* c;             // [M][N] bf16 or fp32
    int m, n, k;
    int tiles_m, tiles_n;
};

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

template <int BM, int BN, int WGM, int WGN, bool A_F32, bool HAS_AWQ, bool OUT_F32>
__global__ __launch_bounds__(64 * WGM * WGN) void gf4_prefill_kernel(PrefillArgs p) {
    constexpr int NT = 64 * WGM * WGN;
    constexpr int WTM = BM / WGM;      // wave tile
    constexpr int WTN = BN / WGN;
    constexpr int FM = WTM / 16;       // MFMA tiles per wave
    constexpr int FN = WTN / 16;
    constexpr int A_CHUNKS = BM * 8 / NT;               // 8-element A chunks per thread per step
    constexpr int B_SLOTS = (BN * 2 + NT - 1) / NT;     // 4-word W chunks per thread per step
    constexpr int BUF = (BM + BN) * kLdsRow;
    static_assert(BM * 8 % NT == 0 && FM >= 1 && FN >= 1 && WTM % 16 == 0 && WTN % 16 == 0, "tile shape");
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
    const uint32_t* b_src[B_SLOTS];
    int b_lds[B_SLOTS];
    bool b_on[B_SLOTS];
#pragma unroll
    for (int i = 0; i < B_SLOTS; ++i) {
        const int c = tid + i * NT;
        b_on[i] = c < BN * 2;
        const int row = b_on[i] ? (c >> 1) : 0;
        const int half = c & 1;
        const int gn = min(n0 + row, p.n - 1);
        b_src[i] = p.w + (size_t)gn * words_per_row + half * 4;
        b_lds[i] = BM * kLdsRow + row * kLdsRow + half * 64;
    }

    uint4_t a_reg[A_CHUNKS][A_F32 ? 2 : 1];
    uint4_t b_reg[B_SLOTS];

    auto load_step = [&](int kt) {
        const int k0 = kt * kBK;
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            if constexpr (A_F32) {
                a_reg[i][0] = *reinterpret_cast<const uint4_t*>(a_src[i] + (size_t)k0 * 4);
                a_reg[i][1] = *reinterpret_cast<const uint4_t*>(a_src[i] + (size_t)k0 * 4 + 16);
            } else {
                a_reg[i][0] = *reinterpret_cast<const uint4_t*>(a_src[i] + (size_t)k0 * 2);
            }
        }
#pragma unroll
        for (int i = 0; i < B_SLOTS; ++i)
            if (b_on[i]) b_reg[i] = load_stream16(b_src[i] + (k0 >> 3));
    };

    auto store_step = [&](int kt, uint8_t* buf) {
        const int k0 = kt * kBK;
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            float v[8];
            if constexpr (A_F32) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // element copies first: bit_cast of a vector-element lvalue reads element 0
                    const uint32_t lo = a_reg[i][0][j];
                    const uint32_t hi = a_reg[i][1][j];
                    v[j] = __builtin_bit_cast(float, lo);
                    v[4 + j] = __builtin_bit_cast(float, hi);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    v[2 * j] = bf16_lo(a_reg[i][0][j]);
                    v[2 * j + 1] = bf16_hi(a_reg[i][0][j]);
                }
            }
            uint4_t out;
            if constexpr (HAS_AWQ) {
                const float4_t s0 = *reinterpret_cast<const float4_t*>(p.awq + k0 + a_col[i]);
                const float4_t s1 = *reinterpret_cast<const float4_t*>(p.awq + k0 + a_col[i] + 4);
                v[0] *= s0.x; v[1] *= s0.y; v[2] *= s0.z; v[3] *= s0.w;
                v[4] *= s1.x; v[5] *= s1.y; v[6] *= s1.z; v[7] *= s1.w;
                out = uint4_t{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]),
                              pack_bf16(v[6], v[7])};
            } else if constexpr (A_F32) {
                out = uint4_t{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]),
                              pack_bf16(v[6], v[7])};
            } else {
                out = a_reg[i][0];
            }
            *reinterpret_cast<uint4_t*>(buf + a_lds[i]) = out;
        }
#pragma unroll
        for (int i = 0; i < B_SLOTS; ++i) {
            if (!b_on[i]) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<uint4_t*>(buf + b_lds[i] + q * 16) = gf4_word_to_bf16x8(b_reg[i][q]);
        }
    };

    float4_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    const int a_rd = (wm * WTM + (lane & 15)) * kLdsRow + (lane >> 4) * 16;
    const int b_rd = BM * kLdsRow + (wn * WTN + (lane & 15)) * kLdsRow + (lane >> 4) * 16;

    const int KT = K / kBK;
    load_step(0);
    store_step(0, smem);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        uint8_t* cur = smem + (kt & 1) * BUF;
        if (kt + 1 < KT) load_step(kt + 1);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            bf16x8_t af[FM], bfr[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *reinterpret_cast<const bf16x8_t*>(cur + a_rd + i * 16 * kLdsRow + ks * 64);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8_t*>(cur + b_rd + j * 16 * kLdsRow + ks * 64);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < KT) store_step(kt + 1, smem + ((kt + 1) & 1) * BUF);
        __syncthreads();
    }

    // Lane l holds D[4*(l/16) + r][l % 16] of each 16x16 tile.
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int gn = n0 + wn * WTN + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gm = m0 + wm * WTM + i * 16 + (lane >> 4) * 4 + r;
                if (gm < p.m && gn < p.n) {
                    const size_t o = (size_t)gm * p.n + gn;
                    if constexpr (OUT_F32) {
                        static_cast<float*>(p.c)[o] = acc[i][j][r];
                    } else {
                        const uint32_t bits = pack_bf16(acc[i][j][r], 0.0f);
                        static_cast<uint16_t*>(p.c)[o] = (uint16_t)bits;
                    }
                }
            }
        }
    }
}

template <int BM, int BN, int WGM, int WGN>
hipError_t launch_tile(const PrefillArgs& a, bool a_f32, bool has_awq, bool out_f32, hipStream_t s) {
    constexpr int NT = 64 * WGM * WGN;
    const size_t lds = 2 * (size_t)(BM + BN) * kLdsRow;
    PrefillArgs p = a;
    p.tiles_m = (a.m + BM - 1) / BM;
    p.tiles_n = (a.n + BN - 1) / BN;
    const dim3 grid(p.tiles_m * p.tiles_n);
#define QW35_PF(AF, AW, OF)                                                                              \
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

}  // namespace

hipError_t launch_gf4_prefill(const void* w, int rows, int k, const void* a, int a_f32, const float* awq, void* c,
                              int m, int out_f32, hipStream_t stream) {
    PrefillArgs p{};
    p.w = static_cast<const uint32_t*>(w);
    p.a = a;
    p.awq = awq;
    p.c = c;
    p.m = m;
    p.n = rows;
    p.k = k;
    const bool af = a_f32 != 0, aw = awq != nullptr, of = out_f32 != 0;
    // Largest tile that still gives every CU a block.
    const long cus = num_cus();
    auto tiles = [&](int bm, int bn) { return (long)((m + bm - 1) / bm) * ((rows + bn - 1) / bn); };
    if (tiles(256, 128) >= cus) return launch_tile<256, 128, 2, 2>(p, af, aw, of, stream);
    if (tiles(128, 128) >= cus) return launch_tile<128, 128, 2, 2>(p, af, aw, of, stream);
    return launch_tile<64, 64, 2, 2>(p, af, aw, of, stream);
}

}  // namespace qw35
