// q8_0, Q4_K, Q5_K, Q6_K and GF4 decode GEMV / fused gate-up-SwiGLU for gfx950, batch 1..8, on MFMA.
//
//   y[b][r] (+)= sum_k W[r][k] * a[k] * x[b][k]
//
// Reference kernels replaced:
//   qw35_decode_matmul_q8_0{,_residual}_f32      (qw35-server/src/metal/qw35_matvec.metal:630-683)
//   qw35_decode_matmul_q4_k_2row{,_residual}_f32 (qw35-server/src/metal/qw35_matvec.metal:171-353)
//   qw35_decode_matmul_q5_k_2row_f32             (qw35-server/src/metal/qw35_matvec.metal:355-456)
//   qw35_decode_matmul_gf4_2row{,_residual}_f32, qw35_ffn_gate_up_swiglu_gf4_f32
//                                                (qw35-server/src/metal/qw35_gf4.metal:62-136,209-246)
//
// Same structure as the GF4 kernel: a workgroup covers 16*RT rows with KS
// waves splitting K into 256-column chunks; raw tensor bytes arrive as
// coalesced 16-byte segments, pass through a per-wave LDS transpose, and each
// lane then reads the bytes of its MFMA operand.  v_mfma_f32_16x16x32_f16:
//   * B (weights): lane l holds 8 consecutive k of weight row n = l % 16 of one
//     32-element block, as exact fp16 integers (q8_0: int8 q; Q4_K: sc_j * q);
//   * A (activations): row 2b = fp16 hi, row 2b+1 = fp16 lo of awq*x of batch
//     row b, scaled per chunk by a power of two (max |v| in [2^13, 2^14));
//   * q8_0 (qw35_types.metal:24-36): one MFMA per 32-element block with a zero
//     accumulator gives the block partial, scaled in fp32: y += d * sum q x;
//   * Q4_K (qw35_matvec.metal:2-38) and Q5_K (qw35_matvec.metal:40-62,355-456;
//     fifth code bit from qh): the 6-bit sub-block scale rides in the fp16
//     operand, so the super-block's eight MFMAs accumulate in one register
//     set and y += d * sum_j sc_j sum q x - dmin * sum_j m_j sum x;
//     the chunk's inverse activation scale is folded into the last multiply.
//
// Byte -> fp16 integer decode (exact, integers below 2048):
//   int8 q:   perm into 0x64XX halves after flipping the sign bit -> 1152 + q,
//             then one v_pk_add_f16 of -1152;
//   nibble q: mask (and shift) -> 0x64XX halves -> 1024 + q, then v_pk_add_f16
//             of -1024, or (Q4_K) v_pk_fma_f16 (1024 + q) * sc - 1024 sc = sc q.
// GF4 words carry their scale inside the exact fp16 operand (gf4_decode.h), so a
// chunk's eight MFMAs accumulate in one register set; lane group kq takes words
// 8kq..8kq+7 of a row (two 16-byte LDS reads) and the activation operand
// follows that k order and the (0,4)(1,5)(2,6)(3,7) pairing within each word.
//
// Q6_K (qw35_types.metal:17-22; GEMV qw35_decode_matmul_q6_k_llama_f32,
// qw35_matvec.metal:458-542): a 210-byte super-block per 256 columns, so a
// chunk starts at byte 210c of the row, 2-byte aligned; it is loaded as the 14
// aligned 16-byte segments that cover it and realigned in registers
// (v_alignbyte).  Its 16 sub-blocks of 16 weights each have an int8 scale, so
// the contraction runs on v_mfma_f32_16x16x16_f16, one MFMA per sub-block:
//   B: the 6-bit code (ql nibble | qh 2 bits << 4) -> exact fp16 q - 32;
//   y += d * sum_s sc_s * sum (q - 32) x  (sc_s applied in fp32 per sub-block,
//   four independent MFMAs before their epilogues, d once per chunk).
//
// Greedy head (qw35_output_q6_k_argmax_partials_16row_f32 +
// qw35_output_argmax_reduce_partials_f32, qw35_output.metal:2-182): with
// GemvArgs::am_token set, the workgroup keeps the largest result of its rows
// per batch row instead of writing y (ties to the smaller row id, NaN never
// chosen), and argmax_reduce_kernel reduces those partials.
#pragma once

#include "gf4_decode.h"
#include "qw35_device.h"
#include "qw35_kernels.h"

#include <stdio.h>

#include <type_traits>
namespace qw35 {

// Per-codec launchers of the chunked kernel (kq_<codec>.hip, kq_<codec>_swiglu.hip).
hipError_t kq_q8_0_plain(const GemvArgs& a, hipStream_t stream);
hipError_t kq_q8_0_swiglu(const GemvArgs& a, hipStream_t stream);
hipError_t kq_q4_k_plain(const GemvArgs& a, hipStream_t stream);
hipError_t kq_q4_k_swiglu(const GemvArgs& a, hipStream_t stream);
hipError_t kq_q5_k_plain(const GemvArgs& a, hipStream_t stream);
hipError_t kq_q5_k_swiglu(const GemvArgs& a, hipStream_t stream);
hipError_t kq_gf2_plain(const GemvArgs& a, hipStream_t stream);
hipError_t kq_gf2_swiglu(const GemvArgs& a, hipStream_t stream);
hipError_t kq_gf4_plain(const GemvArgs& a, hipStream_t stream);
hipError_t kq_gf4_swiglu(const GemvArgs& a, hipStream_t stream);

namespace {


constexpr int kFmtQ8 = 0;
constexpr int kFmtQ4K = 1;
constexpr int kFmtGF4 = 2;
constexpr int kFmtQ6K = 3;
constexpr int kFmtQ5K = 4;
constexpr int kFmtGF2 = 5;

template <int FMT>
struct Fmt;
template <>
struct Fmt<kFmtQ8> {
    static constexpr int kChunkBytes = 272;  // 8 blocks of 34 bytes = 256 columns
    static constexpr int kSegs = 17;         // 16-byte segments per row chunk
    static constexpr int kStride = 288;      // LDS bytes per transposed row (16-byte pad)
    static constexpr int kTypeId = 8;
};
template <>
struct Fmt<kFmtQ4K> {
    static constexpr int kChunkBytes = 144;  // one super-block = 256 columns
    static constexpr int kSegs = 9;
    static constexpr int kStride = 160;
    static constexpr int kTypeId = 12;
};

template <>
struct Fmt<kFmtGF4> {
    static constexpr int kChunkBytes = 128;  // 32 words = 256 columns
    static constexpr int kSegs = 8;
    static constexpr int kStride = 144;
    static constexpr int kTypeId = 100;
};
template <>
struct Fmt<kFmtQ5K> {
    static constexpr int kChunkBytes = 176;  // one super-block = 256 columns
    static constexpr int kSegs = 11;
    static constexpr int kStride = 192;
    static constexpr int kTypeId = 13;
};
template <>
struct Fmt<kFmtGF2> {
    static constexpr int kChunkBytes = 80;  // 16 code words + 16 scale bytes = 256 columns
    static constexpr int kSegs = 5;
    static constexpr int kStride = 96;
    static constexpr int kTypeId = 101;
};
template <>
struct Fmt<kFmtQ6K> {
    static constexpr int kChunkBytes = 210;  // one super-block = 256 columns
    static constexpr int kSegs = 14;         // aligned segments covering bytes [210c, 210c + 210)
    // No pad (2-way bank conflicts on the transposed reads) so that two 16-wave
    // workgroups fit a CU's LDS; the 2-byte realignment of d may read 4 bytes
    // past a row, still inside the wave's block (the activation buffer follows).
    static constexpr int kStride = 224;
    static constexpr int kTypeId = 14;
};

// Byte offset of chunk c's first loaded segment within its row (16-byte
// aligned), and of the chunk's data within that segment (Q6_K only).
template <int FMT>
__device__ __forceinline__ size_t chunk_seg_base(int c) {
    if constexpr (FMT == kFmtQ6K) return (size_t)(c * 210) & ~(size_t)15;
    return (size_t)c * Fmt<FMT>::kChunkBytes;
}

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

// Largest (value, id) under the reference's rule: a candidate wins when it is
// larger, or equal with a smaller id; NaN values enter as (-inf, 0xFFFFFFFF).
__device__ __forceinline__ void argmax_take(float& v, uint32_t& id, float ov, uint32_t oid) {
    if (ov > v || (ov == v && oid < id)) {
        v = ov;
        id = oid;
    }
}

__device__ __forceinline__ void wave_argmax(float& v, uint32_t& id) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(v, o);
        const uint32_t oid = (uint32_t)__shfl_xor((int)id, o);
        argmax_take(v, id, ov, oid);
    }
}

template <int N>
__device__ __forceinline__ void kq_wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <int N, typename F>
__device__ __forceinline__ void kq_static_for(F&& f) {
    if constexpr (N > 0) {
        kq_static_for<N - 1>(f);
        f(std::integral_constant<int, N - 1>{});
    }
}

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// 4 signed bytes -> 2 fp16 pairs (q0,q1), (q2,q3), exact.
__device__ __forceinline__ void s8x4_to_h(uint32_t w, const half2_t bias, uint32_t& p0, uint32_t& p1) {
    const uint32_t t = w ^ 0x80808080u;
    p0 = as_u32(as_half2(__builtin_amdgcn_perm(0x64646464u, t, 0x04010400u)) + bias);
    p1 = as_u32(as_half2(__builtin_amdgcn_perm(0x64646464u, t, 0x04030402u)) + bias);
}

// 4 nibbles (one per byte, already masked) -> 2 fp16 pairs, exact.
__device__ __forceinline__ void u4x4_to_h(uint32_t t, const half2_t bias, uint32_t& p0, uint32_t& p1) {
    p0 = as_u32(as_half2(__builtin_amdgcn_perm(0x64646464u, t, 0x04010400u)) + bias);
    p1 = as_u32(as_half2(__builtin_amdgcn_perm(0x64646464u, t, 0x04030402u)) + bias);
}

typedef uint32_t uint2_t_ __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

// Per-wave LDS block: one transpose buffer (16 rows of a chunk), one activation
// buffer (2*NB rows x 264 halves: one chunk, fp16 hi/lo), a zero row, and
// (Q4_K) the per-sub-block sums of the scaled activations [NB][8].  A wave's
// LDS operations complete in order, so one buffer of each suffices.
template <int FMT, int NB>
struct KqLds {
    static constexpr int kXpose = 16 * Fmt<FMT>::kStride;
    static constexpr int kActStride = 264;  // halves per activation row
    static constexpr int kAct = 2 * NB * kActStride * 2;
    static constexpr int kSx = (FMT == kFmtQ4K || FMT == kFmtQ5K) ? NB * 8 * 4 : 0;
    static constexpr int kXposeOff = 0;
    static constexpr int kActOff = kXpose;
    static constexpr int kZeroOff = kActOff + kAct;
    static constexpr int kSxOff = kZeroOff + 128;
    static constexpr int kBytes = kSxOff + kSx;
};

// Wave w owns chunks w, w + KS, ..., w + (CPW-1)*KS of all RT row tiles, and,
// when the K slice is longer than KS*CPW chunks, the same chunks of each further
// round of KS*CPW.  So the KS waves of a workgroup load KS adjacent chunks at a
// time: a 128-byte line shared by two adjacent chunks (row chunks of 144, 176,
// 210 and 272 bytes for Q4_K, Q5_K, Q6_K and q8_0) is read by two waves at
// about the same time and comes from L2 once, where a wave walking CPW adjacent
// chunks of its own read it again a chunk later, often after L2 had dropped it
// (same box: Q4_K 248320 x 4096 b8 188.8 -> 180.7 us, q8_0 12352 x 4096 b8
// 19.6 -> 19.0 us, Q4_K 4096 x 12288 b1 10.0 -> 9.5 us).  Loads run P chunks
// ahead within a round: chunk c's activations and weight segments are issued
// (in that order) when chunk c-P has been consumed, into register slot c % P.
template <int FMT, int NB, int RT, int KS, int CPW, int P, bool SWIGLU, bool HAS_AWQ, bool ROUNDS>
__device__ __forceinline__ void kq_gemv_body(GemvArgs args) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    using F = Fmt<FMT>;
    using L = KqLds<FMT, NB>;
    constexpr int NM = SWIGLU ? 2 : 1;
    constexpr int LPT = (16 * F::kSegs + 63) / 64;  // 16-byte weight loads per lane per tile
    constexpr int WPC = RT * NM * LPT;                // weight loads per chunk
    // GF4 reads each activation row as two 8-byte pieces per lane (the column
    // pairing of its operand, see issue()); the other formats one 16-byte piece.
    constexpr int XL = FMT == kFmtGF4 ? 2 : 1;
    constexpr int LPC = XL * (NB + (HAS_AWQ ? 1 : 0)) + WPC;  // loads per chunk
    static_assert(P >= 1 && P <= CPW && P * LPC <= 60, "vmcnt budget");
    const int k = args.k;
    const int n_batch = args.n_batch;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15;
    const int kq = lane >> 4;
    // Segment of this workgroup (uniform): its matrix, output and row count.
    const void* wmat = args.w;
    float* yout = args.y;
    int rows = args.rows;
    // K split: consecutive workgroups take the splits of one row group.
    const int splits = args.splits > 1 ? args.splits : 1;
    const int split = (int)blockIdx.x % splits;
    const int group = (int)blockIdx.x / splits;
    int blk = group;
    if (args.n_seg > 1) {
        int seg = 0;
#pragma unroll
        for (int s = 0; s < kMaxSegments - 1; ++s) {
            const int tiles = (args.seg_rows[seg] + 16 * RT - 1) / (16 * RT);
            if (seg + 1 < args.n_seg && blk >= tiles) {
                blk -= tiles;
                ++seg;
            }
        }
        wmat = args.seg_w[seg];
        yout = args.seg_y[seg];
        rows = args.seg_rows[seg];
    }
    const int row0 = blk * 16 * RT;
    const int chunks = k >> 8;
    const size_t row_bytes = (size_t)chunks * F::kChunkBytes;
    const int cps = chunks / splits;  // chunks of this workgroup's K slice
    const int cbase = split * cps;

    uint8_t* wblk = smem + (size_t)wave * L::kBytes;
    // Wave w's partials [RT][NM][NB][16] go to the start of its own LDS block
    // once its last chunk is done (no other wave touches that block).
    static_assert(RT * NM * NB * 16 * 4 <= L::kBytes, "partials fit a wave's block");
    auto part = [&](int w, int t, int m, int b, int nn) -> float& {
        return reinterpret_cast<float*>(smem + (size_t)w * L::kBytes)[((t * NM + m) * NB + b) * 16 + nn];
    };
    if (lane < 32) reinterpret_cast<uint32_t*>(wblk + L::kZeroOff)[lane] = 0u;
    _Float16* xs = reinterpret_cast<_Float16*>(wblk + L::kActOff);
    float* sx = reinterpret_cast<float*>(wblk + L::kSxOff);
    uint8_t* xb = wblk + L::kXposeOff;

    // Register slots of the P chunks in flight.
    float4_t xv[P][NB];
    float4_t av[P];
    uint4_t wv[P][RT * NM][LPT];

    // Byte offset of each lane's 16-byte segments from the tile's first row
    // (rows past the matrix re-read its last row); the per-chunk base is uniform.
    uint32_t loff[RT][LPT];
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            int s = lane + 64 * i;
            s = s < 16 * F::kSegs ? s : 0;
            int r = 16 * t + s / F::kSegs;
            r = r < rows - row0 ? r : rows - 1 - row0;
            loff[t][i] = (uint32_t)r * (uint32_t)row_bytes + 16u * (uint32_t)(s % F::kSegs);
        }

    // First chunk of the current round: a workgroup's KS x CPW chunks cover its
    // K slice in rounds, one round unless k is longer than the plan covers.
    int rb = 0;
    auto issue = [&](auto CI) {
        constexpr int c = decltype(CI)::value;
        constexpr int sl = c % P;
        int chunk = rb + c * KS + wave;
        chunk = cbase + (chunk < cps ? chunk : 0);
        const float* xc = args.x + (size_t)chunk * 256;
        if constexpr (FMT == kFmtGF4) {
            // Columns 8g..8g+7 are staged as x0 x4 x1 x5 | x2 x6 x3 x7: lane 2g
            // reads (x0, x1) and (x4, x5), lane 2g + 1 (x2, x3) and (x6, x7).
            const int c0 = 8 * (lane >> 1) + 2 * (lane & 1);
            auto pairs = [&](const float* p) {
                const float2_t lo = *reinterpret_cast<const float2_t*>(p + c0);
                const float2_t hi = *reinterpret_cast<const float2_t*>(p + c0 + 4);
                return float4_t{lo[0], lo[1], hi[0], hi[1]};
            };
#pragma unroll
            for (int b = 0; b < NB; ++b) xv[sl][b] = pairs(xc + (size_t)(b < n_batch ? b : 0) * k);
            if (HAS_AWQ) av[sl] = pairs(args.awq + (size_t)chunk * 256);
        } else {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int bb = b < n_batch ? b : 0;
                xv[sl][b] = *reinterpret_cast<const float4_t*>(xc + (size_t)bb * k + 4 * lane);
            }
            if (HAS_AWQ) av[sl] = *reinterpret_cast<const float4_t*>(args.awq + (size_t)chunk * 256 + 4 * lane);
        }
        // Tile-major issue order (the order the tiles are consumed in), so that
        // tile t can be decoded while the loads of the tiles after it are in flight.
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const uint8_t* wbase = static_cast<const uint8_t*>(m == 0 ? wmat : args.w_up) +
                                       (size_t)row0 * row_bytes + chunk_seg_base<FMT>(chunk);
#pragma unroll
                for (int i = 0; i < LPT; ++i) {
                    if constexpr (FMT == kFmtQ6K) {
                        // Rows of k % 2048 != 0 start 4, 8 or 12 bytes past a 16-byte
                        // boundary (the low bits of loff): the 16-byte segment holding
                        // the chunk's first byte may then be the next one.  Cached like
                        // Q4_K's below: 210-byte chunks share lines across waves.
                        const uint32_t q15 = (uint32_t)(chunk * 210) & 15u;
                        wv[sl][t * NM + m][i] = load_cached16(wbase + ((loff[t][i] + q15) & ~15u));
                    } else {
                        // Q4_K's 144-byte chunks (Q5_K's 176, GF2's) share a 128-byte
                        // line with the next chunk (another wave's): cached loads keep
                        // it for that reader (LM head 248320x4096 b1: Q4_K 136-149 ->
                        // 122-127 us, 1.40x the weight bytes fetched before; Q5_K
                        // 161 -> 152, GF2 116 -> 108, b8 216 -> 207 and 154 -> 143).
                        // Whole-line GF4 chunks stream.  q8_0 loads cached only in the
                        // one-tile shapes with one chunk in flight (4096x4096 b1 / b8
                        // 6.47 / 9.13 -> 6.28 / 8.62 us); its other shapes measured
                        // the same (12352x4096) or 2-6% slower (4096x12288) cached.
                        constexpr bool kCached = FMT == kFmtQ4K || FMT == kFmtQ5K || FMT == kFmtGF2 ||
                                                 (FMT == kFmtQ8 && RT == 1 && P == 1);
                        wv[sl][t * NM + m][i] = kCached ? load_cached16(wbase + loff[t][i])
                                                        : load_stream16(wbase + loff[t][i]);
                    }
                }
        }
        // loads complete in issue order: keep chunk c's ahead of chunk c + 1's
        __builtin_amdgcn_sched_barrier(0);
    };

    kq_static_for<P>([&](auto CI) { issue(CI); });

    const half2_t bias = FMT == kFmtQ8    ? h2(-1152.0f, -1152.0f)
                         : FMT == kFmtQ6K ? h2(-1056.0f, -1056.0f)
                                          : h2(-1024.0f, -1024.0f);
    const Gf4Consts gc = gf4_consts();
    float acc[RT][NM][2];
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[t][m][0] = acc[t][m][1] = 0.0f;

    for (;;) {
        kq_static_for<CPW>([&](auto CI) {
            constexpr int c = decltype(CI)::value;
            constexpr int sl = c % P;
            constexpr int later = (CPW - 1 - c) < (P - 1) ? (CPW - 1 - c) : (P - 1);  // chunks issued after c
            // chunk c's activations (issued before its weights); each tile's weight
            // loads are waited for where the tile is first read
            kq_wait_vmcnt<later * LPC + WPC>();
            const bool live = rb + c * KS + wave < cps;
            if (live) {
                // Stage chunk c's activations: fp16 hi/lo with a per-chunk power-of-two
                // scale.  The NB row maxima are reduced together (wave_max_rows); the
                // scale and its inverse are uniform integer work; hi = fp16(v s) and
                // lo = fp16(v s - hi) are single mixed-precision FMAs (v s is exact).
                float4_t v[NB];
                uint32_t mx[NB];
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    v[b] = xv[sl][b];
                    if (HAS_AWQ) v[b] *= av[sl];
                    mx[b] = __builtin_bit_cast(uint32_t, fmaxf(fmaxf(fabsf(v[b][0]), fabsf(v[b][1])),
                                                               fmaxf(fabsf(v[b][2]), fabsf(v[b][3]))));
                }
                uint32_t smax[NB];
                wave_max_rows<NB>(mx, smax, lane);
                uint32_t isc_bits[NB];
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    float sc, isc;
                    fp16_range_scale_bits(smax[b], sc, isc);
                    isc_bits[b] = __builtin_bit_cast(uint32_t, isc);
                    float e[4] = {v[b][0], v[b][1], v[b][2], v[b][3]};
                    if constexpr (FMT == kFmtGF4) {
                        // (x0, x1, x4, x5) -> x0 x4 x1 x5 (and the odd lane's likewise)
                        e[1] = v[b][2];
                        e[2] = v[b][1];
                    } else if constexpr (FMT == kFmtGF2) {
                        // Columns 16w..16w+15 stored as x0 x8 x1 x9 .. x3 x11 | x4 x12 .. x7 x15
                        // (MFMA k-slots of lane groups 2(w&1), 2(w&1)+1): the lanes holding
                        // columns 0..3 / 4..7 write (x_c, x_c+8) pairs of their first two
                        // columns, the lanes holding 8..11 / 12..15 those of the last two.
                        float u[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q) u[q] = dpp_f32<kDppQuadXor2>(v[b][q]);
                        if (lane & 2) {
                            e[0] = u[2]; e[1] = v[b][2]; e[2] = u[3]; e[3] = v[b][3];
                        } else {
                            e[0] = v[b][0]; e[1] = u[0]; e[2] = v[b][1]; e[3] = u[1];
                        }
                    }
                    // GF2 k-slot of the lane's four values (natural order otherwise)
                    const int apos = FMT == kFmtGF2 ? 32 * (lane >> 3) + 16 * ((lane >> 2) & 1) + 8 * (lane & 1) +
                                                          4 * ((lane >> 1) & 1)
                                                    : 4 * lane;
                    half2_t hi0, hi1, lo0, lo1;
                    hi0.x = (_Float16)__builtin_fmaf(e[0], sc, 0.0f);
                    hi0.y = (_Float16)__builtin_fmaf(e[1], sc, 0.0f);
                    hi1.x = (_Float16)__builtin_fmaf(e[2], sc, 0.0f);
                    hi1.y = (_Float16)__builtin_fmaf(e[3], sc, 0.0f);
                    lo0.x = (_Float16)__builtin_fmaf(e[0], sc, -(float)hi0.x);
                    lo0.y = (_Float16)__builtin_fmaf(e[1], sc, -(float)hi0.y);
                    lo1.x = (_Float16)__builtin_fmaf(e[2], sc, -(float)hi1.x);
                    lo1.y = (_Float16)__builtin_fmaf(e[3], sc, -(float)hi1.y);
                    *reinterpret_cast<uint2_t_*>(xs + (size_t)(2 * b) * L::kActStride + apos) =
                        uint2_t_{as_u32(hi0), as_u32(hi1)};
                    *reinterpret_cast<uint2_t_*>(xs + (size_t)(2 * b + 1) * L::kActStride + apos) =
                        uint2_t_{as_u32(lo0), as_u32(lo1)};
                    if constexpr (FMT == kFmtQ4K || FMT == kFmtQ5K) {
                        // sum of the scaled activations of each 32-column sub-block (8 lanes)
                        float s4 = (v[b][0] + v[b][1]) + (v[b][2] + v[b][3]);
                        s4 += dpp_f32<kDppQuadXor1>(s4);
                        s4 += dpp_f32<kDppQuadXor2>(s4);
                        s4 += dpp_f32<kDppRowHalfMirror>(s4);
                        if ((lane & 7) == 7) sx[b * 8 + (lane >> 3)] = s4 * sc;
                    }
                }
                float inv_sc[2];  // batches 2kq and 2kq+1
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    uint32_t bits = 0x3F800000u;
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        if (b == 2 * kq + jj) bits = isc_bits[b];
                    inv_sc[jj] = __builtin_bit_cast(float, bits);
                }
                const bool a_live = n < 2 * n_batch;
                const _Float16* arow =
                    a_live ? xs + (size_t)n * L::kActStride : reinterpret_cast<const _Float16*>(wblk + L::kZeroOff);
                const int a_step = a_live ? 32 : 0;
                // GF4: the chunk's activation operands, shared by every tile (words 8kq + j).
                half8_t ga[FMT == kFmtGF4 ? 8 : 1];
                if constexpr (FMT == kFmtGF4) {
                    const _Float16* ap = a_live ? arow + 64 * kq : arow;
#pragma unroll
                    for (int j = 0; j < 8; ++j) ga[j] = *reinterpret_cast<const half8_t*>(ap + (a_live ? 8 * j : 0));
                }

#pragma unroll
                for (int t = 0; t < RT; ++t) {
#pragma unroll
                    for (int m = 0; m < NM; ++m) {
                        // Transpose tile t of matrix m through LDS.
#pragma unroll
                        for (int q = 0; q < LPT; ++q) {
                            const int s = lane + 64 * q;
                            if (s < 16 * F::kSegs)
                                *reinterpret_cast<uint4_t*>(xb + (s / F::kSegs) * F::kStride + 16 * (s % F::kSegs)) =
                                    wv[sl][t * NM + m][q];
                        }
                        wave_sync_lds();
                        const uint8_t* wrow = xb + n * F::kStride;
                        if constexpr (FMT == kFmtGF4) {
                            const uint4_t w0 = *reinterpret_cast<const uint4_t*>(wrow + 32 * kq);
                            const uint4_t w1 = *reinterpret_cast<const uint4_t*>(wrow + 32 * kq + 16);
                            const uint32_t ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                            float4_t dd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int j = 0; j < 8; ++j)
                                dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(ga[j], gf4_word_to_b(ww[j], gc), dd, 0, 0,
                                                                            0);
                            acc[t][m][0] = __builtin_fmaf(inv_sc[0], dd[0] + dd[1], acc[t][m][0]);
                            if constexpr (NB > 1) acc[t][m][1] = __builtin_fmaf(inv_sc[1], dd[2] + dd[3], acc[t][m][1]);
                        } else if constexpr (FMT == kFmtQ8) {
                            // sum_j d_j (hi + lo partial of block j) per batch row; the chunk's
                            // inverse activation scale (a power of two) once at the end
                            float cs0 = 0.0f, cs1 = 0.0f;
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                // qs bytes [2 + 8 kq, +8) of block j: 4-byte aligned for odd j, 2 mod 4 for even j
                                const int off = 34 * j + 2 + 8 * kq;
                                uint32_t d0, d1;
                                if ((j & 1) == 1) {
                                    d0 = *reinterpret_cast<const uint32_t*>(wrow + off);
                                    d1 = *reinterpret_cast<const uint32_t*>(wrow + off + 4);
                                } else {
                                    const uint32_t* base = reinterpret_cast<const uint32_t*>(wrow + off - 2);
                                    const uint32_t e0 = base[0], e1 = base[1], e2 = base[2];
                                    d0 = __builtin_amdgcn_alignbyte(e1, e0, 2);
                                    d1 = __builtin_amdgcn_alignbyte(e2, e1, 2);
                                }
                                const float dsc = (float)*reinterpret_cast<const _Float16*>(wrow + 34 * j);
                                uint32_t b4[4];
                                s8x4_to_h(d0, bias, b4[0], b4[1]);
                                s8x4_to_h(d1, bias, b4[2], b4[3]);
                                const half8_t bop = __builtin_bit_cast(half8_t, uint4_t{b4[0], b4[1], b4[2], b4[3]});
                                const half8_t aop = *reinterpret_cast<const half8_t*>(arow + a_step * j + 8 * kq);
                                const float4_t dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                    aop, bop, float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                                cs0 = __builtin_fmaf(dsc, dd[0] + dd[1], cs0);
                                if constexpr (NB > 1) cs1 = __builtin_fmaf(dsc, dd[2] + dd[3], cs1);
                            }
                            acc[t][m][0] = __builtin_fmaf(inv_sc[0], cs0, acc[t][m][0]);
                            if constexpr (NB > 1) acc[t][m][1] = __builtin_fmaf(inv_sc[1], cs1, acc[t][m][1]);
                        } else if constexpr (FMT == kFmtGF2) {
                            // Step j (32 columns): lane group kq decodes word 2j + (kq >> 1),
                            // codes m and m + 8 for m = 4(kq & 1) .. +3, as pairs in the order
                            // the activations were staged.  Mantissa 2q over 1024:
                            // (1024 + 2q) / 4 - 256.75 = (2q - 3) / 4, exact; times s exact
                            // (5 significant bits); y = 4/3 sum B x.
                            const int hw = kq >> 1;
                            const uint4_t scv = *reinterpret_cast<const uint4_t*>(wrow + 64);
                            const uint32_t scw[4] = {scv.x, scv.y, scv.z, scv.w};
                            // (byte << 8) in both halves: byte hw (even j) or 2 + hw (odd j) of dword j/2
                            const uint32_t sel_even = 0x000C000Cu | (uint32_t)hw * 0x01000100u;
                            const uint32_t sel_odd = 0x020C020Cu | (uint32_t)hw * 0x01000100u;
                            const uint32_t* words = reinterpret_cast<const uint32_t*>(wrow) + hw;
                            const int csh = 8 * (kq & 1);
                            float4_t dd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                const uint32_t cw = words[2 * j] >> csh;
                                const half2_t s2 = as_half2(__builtin_amdgcn_perm(scw[j >> 1], scw[j >> 1],
                                                                                  (j & 1) ? sel_odd : sel_even));
                                const uint32_t pr[4] = {cw << 1, cw >> 1, cw >> 3, cw >> 5};
                                uint32_t b4[4];
#pragma unroll
                                for (int p = 0; p < 4; ++p) {
                                    const half2_t pq = as_half2(and_xor(pr[p], 0x00060006u, 0x64006400u));
                                    b4[p] = as_u32(
                                        __builtin_elementwise_fma(pq, h2(0.25f, 0.25f), h2(-256.75f, -256.75f)) * s2);
                                }
                                const half8_t bop = __builtin_bit_cast(half8_t, uint4_t{b4[0], b4[1], b4[2], b4[3]});
                                const half8_t aop = *reinterpret_cast<const half8_t*>(arow + a_step * j + 8 * kq);
                                dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, dd, 0, 0, 0);
                            }
                            constexpr float kFourThirds = 4.0f / 3.0f;
                            acc[t][m][0] = __builtin_fmaf(inv_sc[0] * kFourThirds, dd[0] + dd[1], acc[t][m][0]);
                            if constexpr (NB > 1)
                                acc[t][m][1] = __builtin_fmaf(inv_sc[1] * kFourThirds, dd[2] + dd[3], acc[t][m][1]);
                        } else if constexpr (FMT == kFmtQ6K) {
                            // The super-block starts `off` bytes into the row buffer: the
                            // chunk's offset past a 16-byte boundary plus the row's own
                            // (n row_bytes mod 16, a multiple of 4; rows past the matrix,
                            // whose results are never stored, take row n's, so reads stay
                            // inside the buffer).  Words are read 4-aligned and, for the
                            // chunks at 2 mod 4, realigned by two bytes.
                            const int q15 = ((cbase + rb + c * KS + wave) * 210) & 15;
                            const int off = (q15 + (int)(((uint32_t)n * (uint32_t)row_bytes) & 15u)) & 15;
                            const uint8_t* sb = wrow + (off & ~3);
                            const _Float16* abase = a_live ? arow + 4 * kq : arow;  // arow: the zero row when !a_live
                            const int astep = a_live ? 16 : 0;
                            auto q6k_chunk = [&](auto ALIGNED) {
                                auto ld = [&](int o) {
                                    const uint32_t* p = reinterpret_cast<const uint32_t*>(sb + o);
                                    if constexpr (decltype(ALIGNED)::value) return p[0];
                                    else return __builtin_amdgcn_alignbyte(p[1], p[0], 2);
                                };
                                const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(ld(208) & 0xFFFFu));
                                uint32_t scw[4];
#pragma unroll
                                for (int q = 0; q < 4; ++q) scw[q] = ld(192 + 4 * q);
                                // sum_s sc_s * sum (q - 32) x in fp32; d and the inverse
                                // activation scale once per chunk.
                                float cs0 = 0.0f, cs1 = 0.0f;
#pragma unroll
                                for (int s4 = 0; s4 < 16; s4 += 4) {
                                    float4_t dd[4];
#pragma unroll
                                    for (int u = 0; u < 4; ++u) {
                                        const int sbk = s4 + u;
                                        const int h = sbk >> 3, g = (sbk & 7) >> 1, p = sbk & 1;
                                        const uint32_t qlw = ld(64 * h + 32 * (g & 1) + 16 * p + 4 * kq);
                                        const uint32_t qhw = ld(128 + 32 * h + 16 * p + 4 * kq);
                                        const uint32_t nib = ((g >> 1) ? (qlw >> 4) : qlw) & 0x0F0F0F0Fu;
                                        const uint32_t qv = nib | (((qhw >> (2 * g)) & 0x03030303u) << 4);
                                        uint32_t b0, b1;
                                        u4x4_to_h(qv, bias, b0, b1);
                                        const half4_t bop = __builtin_bit_cast(half4_t, uint2_t_{b0, b1});
                                        const half4_t aop = *reinterpret_cast<const half4_t*>(abase + astep * sbk);
                                        dd[u] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                                            aop, bop, float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                                    }
#pragma unroll
                                    for (int u = 0; u < 4; ++u) {
                                        const int sbk = s4 + u;
                                        const float scf =
                                            (float)(int)(int8_t)((scw[sbk >> 2] >> (8 * (sbk & 3))) & 0xFFu);
                                        cs0 = __builtin_fmaf(scf, dd[u][0] + dd[u][1], cs0);
                                        if constexpr (NB > 1) cs1 = __builtin_fmaf(scf, dd[u][2] + dd[u][3], cs1);
                                    }
                                }
                                acc[t][m][0] = __builtin_fmaf(d * inv_sc[0], cs0, acc[t][m][0]);
                                if constexpr (NB > 1) acc[t][m][1] = __builtin_fmaf(d * inv_sc[1], cs1, acc[t][m][1]);
                            };
                            if ((q15 & 3) == 0)  // off & 3 == q15 & 3 on every lane
                                q6k_chunk(std::true_type{});
                            else
                                q6k_chunk(std::false_type{});
                        } else {  // Q4_K, Q5_K
                            const uint4_t hd = *reinterpret_cast<const uint4_t*>(wrow);
                            const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)hd.x);
                            const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hd.x >> 16));
                            // 6-bit scales and mins of the 8 sub-blocks, one per byte (get_scale_min_k4).
                            const uint32_t sc_lo = hd.y & 0x3F3F3F3Fu;
                            const uint32_t mn_lo = hd.z & 0x3F3F3F3Fu;
                            const uint32_t sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
                            const uint32_t mn_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
                            // batches past NB read row NB-1 (their results are never stored)
                            const int b0 = min(2 * kq, NB - 1), b1 = min(2 * kq + 1, NB - 1);
                            const float4_t sxa = *reinterpret_cast<const float4_t*>(sx + b0 * 8);
                            const float4_t sxb = *reinterpret_cast<const float4_t*>(sx + b0 * 8 + 4);
                            const float4_t sxc = *reinterpret_cast<const float4_t*>(sx + b1 * 8);
                            const float4_t sxd = *reinterpret_cast<const float4_t*>(sx + b1 * 8 + 4);
                            const float sx0[8] = {sxa[0], sxa[1], sxa[2], sxa[3], sxb[0], sxb[1], sxb[2], sxb[3]};
                            const float sx1[8] = {sxc[0], sxc[1], sxc[2], sxc[3], sxd[0], sxd[1], sxd[2], sxd[3]};
                            // Q4_K's odd sub-blocks (the high nibbles) are decoded in place:
                            // the masked byte 16q under exponent byte 0x54 is the fp16 64 + q
                            // (ulp 1/16 at 64), which saves the shift of the low-nibble path.
                            constexpr bool kHiInPlace = FMT == kFmtQ4K;
                            // Sub-block scales as exact fp16 pairs (sc_2i, sc_2i+1) and the
                            // bias multiples of their biased codes: -1024 sc (1024 + q) and, for
                            // in-place high nibbles, -64 sc (64 + q); |sc| < 64, so both are exact.
                            half2_t scp[4], nbp[4];
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const uint32_t w = i < 2 ? sc_lo : sc_hi;
                                scp[i] = as_half2(__builtin_amdgcn_perm(0x64646464u, w,
                                                                        (i & 1) ? 0x04030402u : 0x04010400u)) +
                                         h2(-1024.0f, -1024.0f);
                                nbp[i] = scp[i] * (kHiInPlace ? h2(-1024.0f, -64.0f) : h2(-1024.0f, -1024.0f));
                            }
                            // B = sc_j * q as one fused multiply-add of the biased code:
                            // (1024 + q) sc - 1024 sc = sc q <= 63 * 31, exact (64 + q likewise);
                            // the eight MFMAs then accumulate sum_j sc_j sum q x in one register set.
                            // Q5_K: bit j of qh byte l (bytes 8kq.. of this lane) is bit 4 of q.
                            constexpr int kQs = FMT == kFmtQ5K ? 48 : 16;
                            const uint2_t_ qh = FMT == kFmtQ5K ? *reinterpret_cast<const uint2_t_*>(wrow + 16 + 8 * kq)
                                                               : uint2_t_{0u, 0u};
                            float4_t dd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int cc = 0; cc < 4; ++cc) {
                                const uint2_t_ qd = *reinterpret_cast<const uint2_t_*>(wrow + kQs + 32 * cc + 8 * kq);
#pragma unroll
                                for (int hi = 0; hi < 2; ++hi) {
                                    const int j = 2 * cc + hi;
                                    const bool in_place = kHiInPlace && hi;
                                    const uint32_t ebase = in_place ? 0x54545454u : 0x64646464u;
                                    uint32_t t0 = in_place ? qd.x & 0xF0F0F0F0u : (hi ? (qd.x >> 4) : qd.x) & 0x0F0F0F0Fu;
                                    uint32_t t1 = in_place ? qd.y & 0xF0F0F0F0u : (hi ? (qd.y >> 4) : qd.y) & 0x0F0F0F0Fu;
                                    if constexpr (FMT == kFmtQ5K) {
                                        const uint32_t h0 = j <= 4 ? qh.x << (4 - j) : qh.x >> (j - 4);
                                        const uint32_t h1 = j <= 4 ? qh.y << (4 - j) : qh.y >> (j - 4);
                                        t0 |= h0 & 0x10101010u;
                                        t1 |= h1 & 0x10101010u;
                                    }
                                    const half2_t sp = scp[j >> 1], np = nbp[j >> 1];
                                    const half2_t s2 = (j & 1) ? half2_t{sp.y, sp.y} : half2_t{sp.x, sp.x};
                                    const half2_t n2 = (j & 1) ? half2_t{np.y, np.y} : half2_t{np.x, np.x};
                                    uint32_t b4[4];
                                    b4[0] = as_u32(__builtin_elementwise_fma(
                                        as_half2(__builtin_amdgcn_perm(ebase, t0, 0x04010400u)), s2, n2));
                                    b4[1] = as_u32(__builtin_elementwise_fma(
                                        as_half2(__builtin_amdgcn_perm(ebase, t0, 0x04030402u)), s2, n2));
                                    b4[2] = as_u32(__builtin_elementwise_fma(
                                        as_half2(__builtin_amdgcn_perm(ebase, t1, 0x04010400u)), s2, n2));
                                    b4[3] = as_u32(__builtin_elementwise_fma(
                                        as_half2(__builtin_amdgcn_perm(ebase, t1, 0x04030402u)), s2, n2));
                                    const half8_t bop =
                                        __builtin_bit_cast(half8_t, uint4_t{b4[0], b4[1], b4[2], b4[3]});
                                    const half8_t aop = *reinterpret_cast<const half8_t*>(arow + a_step * j + 8 * kq);
                                    dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, dd, 0, 0, 0);
                                }
                            }
                            // y += d sum_j sc_j sum q x - dmin sum_j m_j sum x
                            float ms0 = 0.0f, ms1 = 0.0f;
                            if constexpr (NB == 1) {
                                // The four lane groups hold the same batch row: group kq takes
                                // sub-blocks 2kq and 2kq + 1, and the groups' sums are added.
                                const uint32_t mnw = (kq < 2 ? mn_lo : mn_hi) >> (16 * (kq & 1));
                                const float2_t s2x = *reinterpret_cast<const float2_t*>(sx + 2 * kq);
                                float pm = __builtin_fmaf((float)((mnw >> 8) & 0xFFu), s2x[1],
                                                          (float)(mnw & 0xFFu) * s2x[0]);
                                pm += __shfl_xor(pm, 16);
                                ms0 = pm + __shfl_xor(pm, 32);
                            } else {
#pragma unroll
                                for (int j = 0; j < 8; ++j) {
                                    const uint32_t mnw = j < 4 ? mn_lo : mn_hi;
                                    const float mnj = (float)((mnw >> (8 * (j & 3))) & 0xFFu);
                                    ms0 = __builtin_fmaf(mnj, sx0[j], ms0);
                                    ms1 = __builtin_fmaf(mnj, sx1[j], ms1);
                                }
                            }
                            const float v0 = __builtin_fmaf(-dmin, ms0, d * (dd[0] + dd[1]));
                            acc[t][m][0] = __builtin_fmaf(inv_sc[0], v0, acc[t][m][0]);
                            if constexpr (NB > 1) {
                                const float v1 = __builtin_fmaf(-dmin, ms1, d * (dd[2] + dd[3]));
                                acc[t][m][1] = __builtin_fmaf(inv_sc[1], v1, acc[t][m][1]);
                            }
                        }
                        // The next tile (or chunk) rewrites the transpose and activation buffers.
                        wave_sync_lds();
                    }
                }
            }
            if constexpr (c + P < CPW) issue(std::integral_constant<int, c + P>{});
        });
        if constexpr (!ROUNDS) break;
        rb += KS * CPW;
        if (rb >= cps) break;
        kq_static_for<P>([&](auto CI) { issue(CI); });
    }

    // Partials of the KS waves meet in LDS; lane group kq holds batches 2kq, 2kq+1.
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int b = 2 * kq + jj;
                if (b < NB) part(wave, t, m, b, n) = acc[t][m][jj];
            }
    __syncthreads();
    if (args.am_token) {
        // Greedy head: wave b' reduces batch rows b', b' + KS, ...; lane l takes
        // rows l, l + 64, ... of the workgroup (same sums as the y path).
        for (int b = wave; b < n_batch; b += KS) {
            float best = -__builtin_inff();
            uint32_t best_id = 0xFFFFFFFFu;
            for (int o = lane; o < RT * 16; o += 64) {
                const int t = o >> 4, nn = o & 15;
                const int r = row0 + o;
                float sum = 0.0f;
#pragma unroll
                for (int w = 0; w < KS; ++w) sum += part(w, t, 0, b, nn);
                if (r < rows && !__builtin_isnan(sum)) argmax_take(best, best_id, sum, (uint32_t)r);
            }
            wave_argmax(best, best_id);
            if (lane == 0) {
                args.am_logit[(size_t)blockIdx.x * n_batch + b] = best;
                args.am_token[(size_t)blockIdx.x * n_batch + b] = best_id;
            }
        }
        return;
    }
    constexpr int PART = RT * NB * 16 * NM;  // floats of one workgroup's partial
    if (splits > 1) {
        // This workgroup's partial over its K slice goes to the workspace with
        // agent-coherent stores.  After the workgroup barrier, thread 0 moves
        // the row group's counter with an agent-scope release add, which
        // orders the workgroup's partial stores (ordered before it by the
        // barrier) before the add, device-wide.  The adds on one counter form
        // a release sequence, so the workgroup that moves it last, having read
        // the value the others' adds produced, synchronises with all of them
        // through an agent-scope acquire fence and then reads their partials.
        // Only that workgroup pays for the acquire (an invalidation of its
        // XCD's caches): as an acq_rel add on every workgroup it cost 2.5 us
        // per split launch (GF4 4096x12288 batch 8: 12.7 -> 15.5 us).  The last
        // workgroup sums the group's partials in split order (the same order
        // whichever arrives last) and resets the counter for the next launch;
        // nothing waits.
        float* mine = args.ks_part + (size_t)blockIdx.x * PART;
        for (int o = threadIdx.x; o < RT * NB * 16; o += 64 * KS) {
            const int t = o / (NB * 16);
            const int b = (o / 16) % NB;
            const int nn = o & 15;
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                float sum = 0.0f;
#pragma unroll
                for (int w = 0; w < KS; ++w) sum += part(w, t, m, b, nn);
                __hip_atomic_store(mine + o * NM + m, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        kq_wait_vmcnt<0>();
        __shared__ uint32_t last_arrival;
        __syncthreads();
        if (threadIdx.x == 0) {
            const uint32_t prev =
                __hip_atomic_fetch_add(args.ks_count + group, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            last_arrival = prev == (uint32_t)(splits - 1);
            if (last_arrival) {
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                __hip_atomic_store(args.ks_count + group, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __syncthreads();
        if (!last_arrival) return;
        const float* first = args.ks_part + (size_t)(blockIdx.x - split) * PART;
        for (int o = threadIdx.x; o < RT * NB * 16; o += 64 * KS) {
            const int t = o / (NB * 16);
            const int b = (o / 16) % NB;
            const int nn = o & 15;
            const int r = row0 + 16 * t + nn;
            float tot[NM];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                float sum = 0.0f;
                for (int sp = 0; sp < splits; ++sp)
                    sum += __hip_atomic_load(first + (size_t)sp * PART + o * NM + m, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
                tot[m] = sum;
            }
            if (r < rows && b < n_batch) {
                float* yp = yout + (size_t)b * rows + r;
                float v = SWIGLU ? silu(tot[0]) * tot[NM - 1] : tot[0];
                if (args.residual) v += *yp;
                *yp = v;
            }
        }
        return;
    }
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
            for (int w = 0; w < KS; ++w) sum += part(w, t, m, b, nn);
            tot[m] = sum;
        }
        if (r < rows && b < n_batch) {
            float* yp = yout + (size_t)b * rows + r;
            float v = SWIGLU ? silu(tot[0]) * tot[NM - 1] : tot[0];
            if (args.residual) v += *yp;
            *yp = v;
        }
    }
}

// One round: the plan's KS x CPW chunks cover the K slice.
template <int FMT, int NB, int RT, int KS, int CPW, int P, bool SWIGLU, bool HAS_AWQ>
__global__ __launch_bounds__(64 * KS) void kq_mfma_gemv(GemvArgs args) {
    kq_gemv_body<FMT, NB, RT, KS, CPW, P, SWIGLU, HAS_AWQ, false>(args);
}

// Rows longer than one round covers (k beyond 12288 columns).
template <int FMT, int NB, int RT, int KS, int CPW, int P, bool SWIGLU, bool HAS_AWQ>
__global__ __launch_bounds__(64 * KS) void kq_mfma_gemv_long(GemvArgs args) {
    kq_gemv_body<FMT, NB, RT, KS, CPW, P, SWIGLU, HAS_AWQ, true>(args);
}

struct KqPlan {
    int rt, ks, cpw, p;
    int s = 1;  // K splits across workgroups (needs a workspace)
};

// KS waves x CPW chunks cover k with P chunks in flight per wave; RT row tiles
// per workgroup amortise the per-chunk activation staging over more rows.
// Settings from launch-shape sweeps on MI355X (graph replays, rotated weights),
// e.g. q8_0 12352 x 4096 b8 {4, 8, 2, 1} 21.5 us ({3, 8, 2, 2} 35.9 us);
// q8_0 4096 x 4096 b1 {1, 16, 1, 1} 6.2 us ({1, 8, 2, 2} 7.2 us); Q4_K
// 248320 x 4096 b8 {2, 4, 4, 2} 264 us ({4, 8, 2, 1} 275 us).  Batch-1 heads,
// one sweep on one box: Q4_K {3, 8, 2, 2} 134-136 us ({2, 16, 1, 1} 142 us),
// Q6_K {1, 8, 2, 2} 175 us ({2, 16, 1, 1} 183 us; now two tiles, below), GF2
// {3, 8, 2, 2} 113 us ({2, 16, 1, 1} 119 us); Q5_K keeps {2, 16, 1, 1} 157 us
// ({3, 8, 2, 2} 160 us).
inline KqPlan plan_kq(int fmt, int rows, int k, int nb, bool split_ok = false) {
    const int chunks = k >> 8;
    const int tiles = (rows + 15) / 16;
    // Batch 4..8, k = 12288, at most 256 row tiles (the 9B's down projection):
    // with one tile per workgroup every workgroup would stage the whole
    // activation batch, so K is split four ways across workgroups of four
    // tiles, twelve waves, one chunk per wave (GF4 b8 13.0-13.7 us, Q4_K 15.7-16.4,
    // against 17.9 / 21.0 unsplit; two-chunk waves or two-tile workgroups
    // 14.6-22 us).  At k = 4096 no split beat the unsplit q8_0 launch.
    if (split_ok && nb >= 4 && tiles <= 256 && chunks == 48) return {4, 12, 1, 1, 4};
    // Longer rows: eight waves of four chunks per round (kq_mfma_gemv_long).
    if (chunks > 48) return {1, 8, 4, 2};
    if (chunks <= 4) return {1, 4, 1, 1};
    if (chunks <= 8) return {1, 8, 1, 1};
    if (chunks <= 16) {
        if (nb >= 4) {
            if (tiles >= 512) {
                if (fmt != kFmtQ8 && fmt != kFmtGF4) {
                    // LM-head sized: at batch 8 four tiles per 4-wave workgroup
                    // (head b8 Q4_K 199 us, Q6_K 278, Q5_K 249, GF2 176; with
                    // {2, 4, 4, 2} 234 / 322 / 261 / 210 us); Q4_K eight tiles
                    // (one sweep on one box: 170.3 us against 173.5 with four,
                    // 175.9 with six; Q6_K 258.7 with eight, 240.3 with four)
                    if (tiles >= 4096 && nb >= 8 && fmt == kFmtQ4K) return {8, 4, 4, 1};
                    if (tiles >= 4096) return nb >= 8 ? KqPlan{4, 4, 4, 1} : KqPlan{2, 4, 4, 2};
                    return {4, 8, 2, 1};
                }
                if (fmt == kFmtQ8) return {4, 8, 2, 1};
                return {3, 8, 2, 2};
            }
            return fmt == kFmtQ8 ? KqPlan{1, 8, 2, 1} : KqPlan{1, 8, 2, 2};
        }
        if (tiles >= 4096) {  // LM-head sized
            if (fmt == kFmtQ4K) return {3, 8, 2, 2};
            // GF2 (cached loads): four tiles per 4-wave workgroup, one sweep on
            // one box: 99.3-100.0 us against 106-113 with {3, 8, 2, 2}
            if (fmt == kFmtGF2) return {4, 4, 4, 1};
            if (fmt == kFmtQ5K) return {2, 16, 1, 1};
            // Q6_K: two tiles (one sweep on one box: 170.9 us, against 176.7
            // with one, 176.9 with {3, 4, 4, 2}, 183.6 with {4, 8, 2, 1})
            if (fmt == kFmtQ6K) return {2, 8, 2, 2};
        }
        if (fmt == kFmtQ8 && tiles < 512) return {1, 16, 1, 1};
        return {1, 8, 2, 2};
    }
    if (chunks <= 32) return {1, 8, 4, 2};
    if (fmt != kFmtQ8 && fmt != kFmtGF4) return nb >= 4 ? KqPlan{1, 12, 4, 2} : KqPlan{1, 16, 3, 2};
    // GF4 4096 x 12288 b8: {1, 12, 4, 2} 17.1 us ({1, 8, 6, 2} 17.9 us, two sweeps)
    if (fmt == kFmtGF4 && nb >= 8) return {1, 12, 4, 2};
    return {1, 8, 6, 2};
}

template <int FMT, int NB, int RT, int KS, int CPW, bool SWIGLU>
size_t kq_lds_bytes() {
    constexpr int NM = SWIGLU ? 2 : 1;
    (void)NM;
    return (size_t)KS * KqLds<FMT, NB>::kBytes;
}

// K-split workspace: kKsCounters row-group counters at its start (the same
// place for every shape, so a launch always finds the counters the previous
// one returned to zero), then the partials (one RT x NB x 16 x NM block per
// workgroup).  Split plans cover at most 256 row tiles, so at most 256 groups.
constexpr int kKsCounters = 256;
constexpr size_t kKsPartOffset = kKsCounters * 4;
inline size_t kq_split_ws_bytes(int groups, int splits, int rt, int nb, int nm) {
    return splits > 1 ? kKsPartOffset + ((size_t)groups * splits * rt * nb * 16 * nm * 4 + 255) / 256 * 256 : 0;
}

template <int FMT, int NB, int RT, int KS, int CPW, int P, bool SWIGLU, bool LONG = false>
hipError_t kq_launch_cfg(const GemvArgs& a0, hipStream_t stream, int splits = 1) {
    const size_t lds = kq_lds_bytes<FMT, NB, RT, KS, CPW, SWIGLU>();
    if (lds > 160 * 1024) return hipErrorInvalidConfiguration;
    GemvArgs a = a0;
    int grid = (a.rows + 16 * RT - 1) / (16 * RT);
    if (a.n_seg > 1) {
        grid = 0;
        for (int s = 0; s < a.n_seg; ++s) grid += (a.seg_rows[s] + 16 * RT - 1) / (16 * RT);
    }
    const int groups = grid;
    // every chunk of K belongs to some wave of some split, in one round or (LONG) several
    if (!LONG && (a.k >> 8) > KS * CPW * splits) return hipErrorInvalidValue;
    const size_t ws_need = kq_split_ws_bytes(groups, splits, RT, NB, SWIGLU ? 2 : 1);
    if (splits > 1 && (a.am_token || !a.ks_ws || a.ks_ws_bytes < ws_need || (a.k >> 8) % splits != 0 ||
                       (!LONG && (a.k >> 8) / splits > KS * CPW) || groups > kKsCounters))
        return hipErrorInvalidValue;
    a.splits = splits;
    if (splits > 1) {
        a.ks_count = static_cast<uint32_t*>(a.ks_ws);
        a.ks_part = reinterpret_cast<float*>(static_cast<uint8_t*>(a.ks_ws) + kKsPartOffset);
        grid *= splits;
    }
    // The greedy head's partial workspace holds argmax_groups() entries per
    // batch row: refuse a launch shape with more workgroups than that.
    if (a.am_token && grid != argmax_groups(Fmt<FMT>::kTypeId, a.rows, a.k, a.n_batch)) return hipErrorInvalidValue;
    if (a.info) {
        snprintf(a.info->name, sizeof a.info->name, "%s<%d, %d, %d, %d, %d, %d, %s, %s>",
                 LONG ? "kq_mfma_gemv_long" : "kq_mfma_gemv", FMT, NB, RT, KS, CPW, P, SWIGLU ? "true" : "false",
                 a.awq ? "true" : "false");
        a.info->grid = (unsigned)grid;
        a.info->block = 64u * KS;
        a.info->lds = (unsigned)lds;
        a.info->splits = (unsigned)splits;
        a.info->ws_bytes = ws_need;
        return hipSuccess;
    }
    if constexpr (LONG) {
        if (a.awq)
            hipLaunchKernelGGL((kq_mfma_gemv_long<FMT, NB, RT, KS, CPW, P, SWIGLU, true>), dim3(grid), dim3(64 * KS),
                               lds, stream, a);
        else
            hipLaunchKernelGGL((kq_mfma_gemv_long<FMT, NB, RT, KS, CPW, P, SWIGLU, false>), dim3(grid),
                               dim3(64 * KS), lds, stream, a);
    } else {
        if (a.awq)
            hipLaunchKernelGGL((kq_mfma_gemv<FMT, NB, RT, KS, CPW, P, SWIGLU, true>), dim3(grid), dim3(64 * KS), lds,
                               stream, a);
        else
            hipLaunchKernelGGL((kq_mfma_gemv<FMT, NB, RT, KS, CPW, P, SWIGLU, false>), dim3(grid), dim3(64 * KS),
                               lds, stream, a);
    }
    return hipGetLastError();
}

// Loads in flight per wave for a configuration (must fit the vmcnt counter).
template <int FMT, int NB, int RT, int P, bool SWIGLU>
constexpr bool kq_fits() {
    constexpr int lpt = (16 * Fmt<FMT>::kSegs + 63) / 64;
    constexpr int xl = FMT == kFmtGF4 ? 2 : 1;
    return P * (xl * (NB + 1) + RT * (SWIGLU ? 2 : 1) * lpt) <= 60;
}

template <int FMT, int NB, bool SWIGLU>
hipError_t kq_launch_nb(const GemvArgs& a, hipStream_t stream) {
    int total_rows = a.rows;
    if (a.n_seg > 1) {
        total_rows = 0;
        for (int s = 0; s < a.n_seg; ++s) total_rows += a.seg_rows[s];
    }
    if ((a.k >> 8) > 48)  // the long-row plan of plan_kq, in rounds of 32 chunks
        return kq_launch_cfg<FMT, NB, 1, 8, 4, (kq_fits<FMT, NB, 1, 2, SWIGLU>() ? 2 : 1), SWIGLU, true>(a, stream);
    KqPlan p = plan_kq(FMT, total_rows, a.k, NB, a.ks_ws != nullptr && !a.am_token);
    if (p.s > 1) {
        int groups = (a.rows + 16 * p.rt - 1) / (16 * p.rt);
        if (a.n_seg > 1) {
            groups = 0;
            for (int s = 0; s < a.n_seg; ++s) groups += (a.seg_rows[s] + 16 * p.rt - 1) / (16 * p.rt);
        }
        if (a.ks_ws_bytes < kq_split_ws_bytes(groups, p.s, p.rt, NB, SWIGLU ? 2 : 1))
            p = plan_kq(FMT, total_rows, a.k, NB, false);
    }
    // Fused gate/up holds two matrices' loads per tile: more than two row tiles
    // per workgroup spill registers, so those take the one-tile shape below.
#define QW35_KQ_PLAN(RT, KS, CPW, P)                                                             \
    if constexpr (kq_fits<FMT, NB, RT, P, SWIGLU>() && (!SWIGLU || RT <= 2)) {                     \
        if (p.rt == RT && p.ks == KS && p.cpw == CPW && p.p == P)                                  \
            return kq_launch_cfg<FMT, NB, RT, KS, CPW, P, SWIGLU>(a, stream, p.s);                 \
    }
    QW35_KQ_PLAN(1, 4, 1, 1)
    QW35_KQ_PLAN(1, 8, 1, 1)
    QW35_KQ_PLAN(1, 8, 2, 2)
    QW35_KQ_PLAN(3, 8, 2, 2)
    QW35_KQ_PLAN(4, 8, 2, 1)
    QW35_KQ_PLAN(1, 8, 4, 2)
    QW35_KQ_PLAN(1, 8, 6, 2)
    if constexpr (FMT == kFmtQ8) {
        if constexpr (NB >= 4) {
            QW35_KQ_PLAN(1, 8, 2, 1)
        } else {
            QW35_KQ_PLAN(1, 16, 1, 1)
        }
    }
    if constexpr (NB == 8 && (FMT == kFmtQ4K || FMT == kFmtQ6K || FMT == kFmtQ5K || FMT == kFmtGF2)) {
        QW35_KQ_PLAN(4, 4, 4, 1)
    }
    if constexpr (NB == 8 && FMT == kFmtQ4K) {
        QW35_KQ_PLAN(8, 4, 4, 1)
    }
    if constexpr (NB <= 2 && FMT == kFmtQ6K) {
        QW35_KQ_PLAN(2, 8, 2, 2)
    }
    if constexpr (NB <= 2 && FMT == kFmtGF2) {
        QW35_KQ_PLAN(4, 4, 4, 1)
    }
    if constexpr (NB == 8 && FMT == kFmtGF4) {
        QW35_KQ_PLAN(1, 12, 4, 2)
    }
    if constexpr (NB >= 4 && !SWIGLU) {  // the K-split plan
        QW35_KQ_PLAN(4, 12, 1, 1)
    }
    if constexpr (FMT == kFmtQ4K || FMT == kFmtQ5K || FMT == kFmtQ6K || FMT == kFmtGF2) {
        if constexpr (NB >= 4) {
            QW35_KQ_PLAN(2, 4, 4, 2)
            QW35_KQ_PLAN(1, 12, 4, 2)
        } else {
            QW35_KQ_PLAN(2, 16, 1, 1)
            QW35_KQ_PLAN(1, 16, 3, 2)
        }
    }
    // Fused gate/up planned with more than two tiles: three tiles with one
    // chunk in flight (half the load registers of the planned shape, so no
    // spills); 12288 rows are then exactly 256 workgroups, one per CU.
    if constexpr (SWIGLU && NB >= 4 && kq_fits<FMT, NB, 3, 1, SWIGLU>()) {
        if (p.rt > 2) return kq_launch_cfg<FMT, NB, 3, 8, 2, 1, SWIGLU>(a, stream);
    }
    // over the load budget or the register budget (fused gate/up): one tile per workgroup
    if (p.rt > 1) return kq_launch_cfg<FMT, NB, 1, 8, 2, (kq_fits<FMT, NB, 1, 2, SWIGLU>() ? 2 : 1), SWIGLU>(a, stream);
#undef QW35_KQ_PLAN
    return hipErrorInvalidValue;
}

template <int FMT, bool SWIGLU>
hipError_t kq_launch_any(const GemvArgs& a, hipStream_t stream) {
    if (a.n_batch == 1) return kq_launch_nb<FMT, 1, SWIGLU>(a, stream);
    if (a.n_batch == 2) return kq_launch_nb<FMT, 2, SWIGLU>(a, stream);
    if (a.n_batch <= 4) return kq_launch_nb<FMT, 4, SWIGLU>(a, stream);
    return kq_launch_nb<FMT, 8, SWIGLU>(a, stream);
}

}  // namespace
}  // namespace qw35
