// Greedy head: the reduction of the per-workgroup (logit, row) partials that
// the chunked GEMV kernels write with GemvArgs::am_token set, and its launcher.
#include "kquant_mfma.h"

namespace qw35 {
namespace {

// Final reduction of the greedy-head partials: block b reduces batch row b.
// Each thread issues kArgmaxLoads loads before comparing, so one pass over
// the partials costs one memory latency (a 248320-row head has 7760 groups).
constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxLoads = 8;

__global__ __launch_bounds__(kArgmaxThreads) void argmax_reduce_kernel(const uint32_t* __restrict__ pt,
                                                                       const float* __restrict__ pv, int n_groups,
                                                                       int n_batch, uint32_t* __restrict__ token,
                                                                       float* __restrict__ logit) {
    __shared__ float sv[kArgmaxThreads / 64];
    __shared__ uint32_t sid[kArgmaxThreads / 64];
    const int b = blockIdx.x;
    float best = -__builtin_inff();
    uint32_t best_id = 0xFFFFFFFFu;
    for (int g0 = threadIdx.x; g0 < n_groups; g0 += kArgmaxThreads * kArgmaxLoads) {
        float v[kArgmaxLoads];
        uint32_t id[kArgmaxLoads];
#pragma unroll
        for (int u = 0; u < kArgmaxLoads; ++u) {
            const int g = g0 + u * kArgmaxThreads;
            v[u] = g < n_groups ? pv[(size_t)g * n_batch + b] : -__builtin_inff();
            id[u] = g < n_groups ? pt[(size_t)g * n_batch + b] : 0xFFFFFFFFu;
        }
#pragma unroll
        for (int u = 0; u < kArgmaxLoads; ++u)
            if (!__builtin_isnan(v[u])) argmax_take(best, best_id, v[u], id[u]);
    }
    wave_argmax(best, best_id);
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = best;
        sid[threadIdx.x >> 6] = best_id;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float v = sv[0];
        uint32_t id = sid[0];
        for (int w = 1; w < kArgmaxThreads / 64; ++w) argmax_take(v, id, sv[w], sid[w]);
        token[b] = id;
        logit[b] = v;
    }
}

int fmt_of(uint32_t type_id) {
    switch (type_id) {
        case kTypeQ8_0: return kFmtQ8;
        case kTypeQ4_K: return kFmtQ4K;
        case kTypeQ5_K: return kFmtQ5K;
        case kTypeGF2: return kFmtGF2;
        case kTypeQ6_K: return kFmtQ6K;
        default: return kFmtGF4;
    }
}
}  // namespace

int argmax_groups(uint32_t type_id, int rows, int k, int n_batch) {
    const int nb = n_batch <= 1 ? 1 : n_batch == 2 ? 2 : n_batch <= 4 ? 4 : 8;
    const KqPlan p = plan_kq(fmt_of(type_id), rows, k, nb);
    return (rows + 16 * p.rt - 1) / (16 * p.rt);
}

hipError_t launch_argmax_gemv(uint32_t type_id, const GemvArgs& a, uint32_t* token, float* logit,
                              hipStream_t stream) {
    if (!a.am_token || !a.am_logit || a.w_up || a.n_seg > 1) return hipErrorInvalidValue;
    hipError_t e;
    switch (type_id) {
        case kTypeQ8_0: e = kq_q8_0_plain(a, stream); break;
        case kTypeQ4_K: e = kq_q4_k_plain(a, stream); break;
        case kTypeQ5_K: e = kq_q5_k_plain(a, stream); break;
        case kTypeGF2: e = kq_gf2_plain(a, stream); break;
        case kTypeQ6_K: e = launch_q6_k_gemv(a, stream); break;
        default: e = kq_gf4_plain(a, stream); break;
    }
    if (e != hipSuccess || a.info) return e;
    const int groups = argmax_groups(type_id, a.rows, a.k, a.n_batch);
    hipLaunchKernelGGL(argmax_reduce_kernel, dim3(a.n_batch), dim3(kArgmaxThreads), 0, stream, a.am_token,
                       a.am_logit, groups, a.n_batch, token, logit);
    return hipGetLastError();
}

}  // namespace qw35
