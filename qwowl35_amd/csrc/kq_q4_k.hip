// Chunked decode GEMV, q4_k, plain (and greedy-head) instantiations (kernel in kquant_mfma.h).
#include "kquant_mfma.h"

namespace qw35 {

hipError_t kq_q4_k_plain(const GemvArgs& a, hipStream_t stream) {
    return kq_launch_any<kFmtQ4K, false>(a, stream);
}

hipError_t launch_q4_k_gemv(const GemvArgs& a, hipStream_t stream) {
    return a.w_up ? kq_q4_k_swiglu(a, stream) : kq_q4_k_plain(a, stream);
}

}  // namespace qw35
