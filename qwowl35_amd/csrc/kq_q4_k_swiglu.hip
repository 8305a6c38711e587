// Chunked decode GEMV, q4_k, fused gate/up/SwiGLU instantiations (kernel in kquant_mfma.h).
#include "kquant_mfma.h"

namespace qw35 {

hipError_t kq_q4_k_swiglu(const GemvArgs& a, hipStream_t stream) {
    return kq_launch_any<kFmtQ4K, true>(a, stream);
}

}  // namespace qw35
