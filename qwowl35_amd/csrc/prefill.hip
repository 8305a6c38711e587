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
//   LDS (double buffered, 16-byte row padding against bank conflicts).  Global
//   loads run two steps ahead in two register stages; a step's conversion (AWQ
//   multiply + RNE for A, GF4 decode for W) follows the MFMAs of the step
//   before it, so one barrier per step suffices.
// * The W tile is the MFMA's first operand: lane l accumulates
//   D[n = 4 (l / 16) + r][m = l % 16], four consecutive outputs of one token
//   row, stored as one 8- or 16-byte vector.
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

template <int BM, int BN, int NT, bool A_F32>
struct StepRegs {
    static constexpr int A_CHUNKS = BM * 8 / NT;  // 8-element A chunks per thread
    static constexpr int WPT = BN * 8 / NT;       // GF4 words per thread
    uint4_t a[A_CHUNKS][A_F32 ? 2 : 1];
    uint32_t b[WPT];
};

template <int BM, int BN, int WGM, int WGN, bool A_F32, bool HAS_AWQ, bool OUT_F32>
// Two waves per SIMD (<= 256 VGPRs): one wave's loads and conversions overlap
// the other's MFMAs.
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
            const uint4_t v = load_stream16(bs);
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
    if (!af && tiles(256, 128) >= cus) return launch_tile<256, 128, 4, 2>(p, af, aw, of, stream);
    if (tiles(128, 128) >= cus) return launch_tile<128, 128, 2, 2>(p, af, aw, of, stream);
    return launch_tile<64, 64, 2, 2>(p, af, aw, of, stream);
}

}  // namespace qw35
