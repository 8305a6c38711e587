// Chunked decode GEMV, q6_k, plain (and greedy-head) instantiations (kernel in kquant_mfma.h).
#include "kquant_mfma.h"

namespace qw35 {

// Q6_K has no fused gate/up form (the reference uses it for the LM head only).
hipError_t launch_q6_k_gemv(const GemvArgs& a, hipStream_t stream) {
    if (a.w_up) return hipErrorInvalidValue;
    return kq_launch_any<kFmtQ6K, false>(a, stream);
}

}  // namespace qw35
