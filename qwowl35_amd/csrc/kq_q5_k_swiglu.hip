// Chunked decode GEMV, q5_k, fused gate/up/SwiGLU instantiations (kernel in kquant_mfma.h).
#include "kquant_mfma.h"

namespace qw35 {

hipError_t kq_q5_k_swiglu(const GemvArgs& a, hipStream_t stream) {
    return kq_launch_any<kFmtQ5K, true>(a, stream);
}

}  // namespace qw35
