// Host-side launch interface of the qw35 HIP kernels (internal to the library;
// the public C ABI is include/qw35_hip.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qw35 {

// GGUF tensor type-ids handled by this library.
constexpr uint32_t kTypeF16 = 1;
constexpr uint32_t kTypeQ8_0 = 8;
constexpr uint32_t kTypeQ4_K = 12;
constexpr uint32_t kTypeQ5_K = 13;
constexpr uint32_t kTypeQ6_K = 14;
constexpr uint32_t kTypeGF4 = 100;
constexpr uint32_t kTypeGF2 = 101;

// Largest decode batch of the GEMV kernels.
constexpr int kMaxDecodeBatch = 8;

// Matrices sharing k, type, activations and batch can share one launch
// (q8_0 / Q4_K kernels): segment s covers the rows of seg_w[s], written to seg_y[s].
constexpr int kMaxSegments = 4;

// Filled instead of launching when GemvArgs::info is set: the kernel
// instantiation as the profiler names it, and its launch shape.
struct LaunchInfo {
    char name[160];
    unsigned grid;
    unsigned block;
    unsigned lds;
    unsigned splits;    // K splits of the launch (1: none)
    uint64_t ws_bytes;  // K-split workspace the launch uses (0: none)
};

struct GemvArgs {
    const void* w;        // raw tensor bytes, row-major, rows x row_bytes
    const float* x;       // [n_batch][k]
    const float* awq;     // [k] or nullptr
    float* y;             // [n_batch][rows]
    const void* w_up;     // second matrix of the fused gate/up/SwiGLU kernel, else nullptr
    int rows;
    int k;
    int n_batch;
    int residual;         // y += result instead of y = result
    int n_seg;            // 0: the single matrix (w, y, rows); 2..kMaxSegments: the segments
    const void* seg_w[kMaxSegments];
    float* seg_y[kMaxSegments];
    int seg_rows[kMaxSegments];
    // Greedy head (q8_0 / Q4_K / Q6_K / GF4 chunked kernel only): when am_token
    // is set, y is not written; each workgroup writes the largest of its rows'
    // results per batch row b (ties to the smaller row, NaN never chosen) to
    // am_logit / am_token[blockIdx.x * n_batch + b].
    uint32_t* am_token;
    float* am_logit;
    // Host pointer: when set, the launchers describe the (first) launch here
    // and launch nothing.
    LaunchInfo* info;
    // K-split workspace (nullable, 256-byte aligned, zero-filled before its
    // first use): with it the chunked kernel's planner may split K across
    // workgroups (partials, then one counter per row group, which the kernel
    // returns to zero).  splits / ks_part / ks_count are set by the launcher.
    void* ks_ws;
    uint64_t ks_ws_bytes;
    int splits;
    float* ks_part;
    uint32_t* ks_count;
};

// Each launcher validates nothing (the C ABI does) and returns the launch status.
hipError_t launch_gf4_gemv(const GemvArgs& a, hipStream_t stream);
hipError_t launch_q8_0_gemv(const GemvArgs& a, hipStream_t stream);
// q8_0 rows of k % 256 != 0 (k % 32 == 0): one wave per row, no greedy head.
hipError_t launch_q8_0_gemv_rows(const GemvArgs& a, hipStream_t stream);
hipError_t launch_q4_k_gemv(const GemvArgs& a, hipStream_t stream);
hipError_t launch_q5_k_gemv(const GemvArgs& a, hipStream_t stream);
hipError_t launch_gf2_gemv(const GemvArgs& a, hipStream_t stream);
hipError_t launch_q6_k_gemv(const GemvArgs& a, hipStream_t stream);

// Greedy head: workgroups of the GEMV launch that launch_argmax_gemv makes for
// (type_id, rows, k, n_batch) -- the number of partials per batch row.
int argmax_groups(uint32_t type_id, int rows, int k, int n_batch);
// GEMV with the argmax epilogue (a.am_token / a.am_logit hold
// argmax_groups(...) * n_batch partials), then the reduction of the partials to
// token[b], logit[b].
hipError_t launch_argmax_gemv(uint32_t type_id, const GemvArgs& a, uint32_t* token, float* logit, hipStream_t stream);
// GF4 on the chunked k-quant kernel structure (rolling prefetch, per-chunk
// activation staging); launch_gf4_gemv picks between the two.
hipError_t launch_gf4_gemv_chunked(const GemvArgs& a, hipStream_t stream);

// Full or row-gathered dequantisation (row_ids == nullptr: all rows), to fp32
// or (f16_out) to fp16 round-to-nearest-even of the same value.
hipError_t launch_dequant(uint32_t type_id, const void* w, int rows, int k, const uint32_t* row_ids,
                          int n_out_rows, void* dst, bool f16_out, hipStream_t stream);

// fp32 [rows][k] -> tensor bytes of type_id (GF4 packer / q8_0 / Q4_K encoders);
// col_scale (nullable) multiplies column c first.
hipError_t launch_quantize(uint32_t type_id, const float* src, int rows, int k, const float* col_scale, void* dst,
                           hipStream_t stream);

// Streaming-read probe over `bytes` (a multiple of 16) of `buf`; sink holds
// stream_read_blocks(bytes) uint32 values.
unsigned stream_read_blocks(uint64_t bytes);
hipError_t launch_stream_read(const void* buf, uint64_t bytes, uint32_t* sink, hipStream_t stream);

// MFMA throughput probe: workgroups x 4 waves x iters x 8 v_mfma_f32_32x32x16_f16
// (32768 flops each); sink holds workgroups * 256 floats.
hipError_t launch_mfma_probe(unsigned workgroups, unsigned iters, float* sink, hipStream_t stream);

// Prefill dequant-matmul of GF4 words, F16 weights or q8_0 blocks (wkind 0, 1, 2):
//   C[m][n] = sum_k v[m][k] * W[n][k],  v = awq[k] * A[m][k] (fp32 product), fp32 accumulation.
// a: [m][k] bf16 (a_f32 == 0) or fp32; c: [m][rows] bf16 RNE (out_f32 == 0) or fp32.
// workspace (nullable for GF4 only; 256-byte aligned, at least
// prefill_min_workspace_bytes(m, rows, k, a_f32)): stage v as fp16 with
// per-token power-of-two scales (fp32 input: an fp16 hi and lo row per token,
// about 22 significant bits) and contract on fp16 MFMA, split over K (fp32
// partials in the workspace) when the tiles alone would leave CUs idle and
// workspace_bytes holds the partials.  Without a workspace (GF4): bf16 MFMA on
// bf16_rne(v), no split.
struct PrefillCfg {
    int bm;      // tokens per block: 256 (F16 / q8_0 weights), 128, 64 or 32
    int fn;      // 32-row weight tiles per wave (4 waves per block): 2 or 4 (4 needs bm >= 64)
    int splits;  // K splits; k / splits must be a multiple of 256
    // 8: the same bm x 256 tile on 8 waves of one 32-row weight tile each
    // (GF4, fn 2 only), two waves per SIMD where a CU gets only one block.
    // 16: only with kh 4 (below).
    int waves = 4;
    // 2 (8-wave tiles only): the 8 waves form two K halves of four waves over
    // a 128-row tile, summed in LDS; splits then counts blocks per K range.
    // 4 (GF4, bm 64, fn 2): four K quarters, of two waves over a 64-row tile
    // (waves 8) or of four over a 128-row tile (waves 16).
    int kh = 1;
};
PrefillCfg plan_prefill_kind(int m, int rows, int k, int wkind, bool a_f32);
PrefillCfg plan_gf4_prefill(int m, int rows, int k, bool a_f32);
size_t gf4_prefill_workspace_bytes(int m, int rows, int k, PrefillCfg cfg, bool a_f32);
// Workspace of the planned launch for bf16 activations, or (with_f32) the
// larger of the bf16 and fp32 ones.
size_t prefill_workspace_bytes(int m, int rows, int k, int wkind, bool with_f32);
// Smallest workspace the staged path accepts (no K split).
size_t prefill_min_workspace_bytes(int m, int rows, int k, bool a_f32);
// Up to kMaxSegments matrices of one weight form and k that read the same
// activations (a mixer's input projections), as one staged launch: the
// weight tiles of all of them form one grid and each writes its own output
// c[s] ([m][rows[s]]).  rows[s] must be multiples of 4; the launch is planned
// for their sum, which the rows argument must equal.
struct PrefillSegs {
    int n = 0;  // 0 or 1: the single matrix (w, c, rows)
    const void* w[kMaxSegments] = {};
    void* c[kMaxSegments] = {};
    int rows[kMaxSegments] = {};
};
// epi (fp32 c with a workspace only): 0 c = r, 1 c += r, 2 c = silu(c) * r.
// info (host pointer, nullable): describe the matmul launch (name, grid,
// block, LDS, splits; ws_bytes the workspace it uses) and launch nothing.
// staged: the workspace already holds these activations staged for this
// weight form (the previous launch on it staged the same a, awq, m, k and
// column order), so the staging pass is not launched again.
hipError_t launch_gf4_prefill_cfg(const void* w, int rows, int k, const void* a, int a_f32, const float* awq,
                                  void* c, int m, int out_f32, void* workspace, PrefillCfg cfg, hipStream_t stream,
                                  int wkind = 0, int epi = 0, LaunchInfo* info = nullptr,
                                  bool staged = false,  // wkind 0 GF4, 1 F16, 2 q8_0, 3 Q4_K
                                  const PrefillSegs* segs = nullptr, const void* w_up = nullptr);
// Planned launch; the workspace is required for F16 and q8_0 weights.
hipError_t launch_prefill(int wkind, const void* w, int rows, int k, const void* a, int a_f32, const float* awq,
                          void* c, int m, int out_f32, void* workspace, size_t workspace_bytes, hipStream_t stream,
                          int epi = 0, LaunchInfo* info = nullptr, bool staged = false,
                          const PrefillSegs* segs = nullptr, const void* w_up = nullptr);
// w_up (with w the gate): c = silu(gate v) * (up v) in one launch, the bits of
// the gate launch (STORE) followed by the up launch (SWIGLU epilogue), where
// prefill_swiglu_fusable says the planned gate launch has the fused form (GF4
// words, fp32 c, a workspace, epi STORE); invalid otherwise.
bool prefill_swiglu_fusable(int wkind, int m, int rows, int k, int a_f32, size_t workspace_bytes);

}  // namespace qw35
