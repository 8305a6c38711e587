// Chunked decode GEMV, gf2, fused gate/up/SwiGLU instantiations (kernel in kquant_mfma.h).
#include "kquant_mfma.h"

namespace qw35 {

hipError_t kq_gf2_swiglu(const GemvArgs& a, hipStream_t stream) {
    return kq_launch_any<kFmtGF2, true>(a, stream);
}

}  // namespace qw35
