// Chunked decode GEMV, gf2, plain (and greedy-head) instantiations (kernel in kquant_mfma.h).
#include "kquant_mfma.h"

namespace qw35 {

hipError_t kq_gf2_plain(const GemvArgs& a, hipStream_t stream) {
    return kq_launch_any<kFmtGF2, false>(a, stream);
}

hipError_t launch_gf2_gemv(const GemvArgs& a, hipStream_t stream) {
    return a.w_up ? kq_gf2_swiglu(a, stream) : kq_gf2_plain(a, stream);
}

}  // namespace qw35
