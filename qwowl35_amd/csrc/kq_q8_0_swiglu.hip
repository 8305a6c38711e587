// Chunked decode GEMV, q8_0, fused gate/up/SwiGLU instantiations (kernel in kquant_mfma.h).
#include "kquant_mfma.h"

namespace qw35 {

hipError_t kq_q8_0_swiglu(const GemvArgs& a, hipStream_t stream) {
    return kq_launch_any<kFmtQ8, true>(a, stream);
}

}  // namespace qw35
