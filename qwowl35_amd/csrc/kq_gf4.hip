// Chunked decode GEMV, gf4, plain (and greedy-head) instantiations (kernel in kquant_mfma.h).
#include "kquant_mfma.h"

namespace qw35 {

hipError_t kq_gf4_plain(const GemvArgs& a, hipStream_t stream) {
    return kq_launch_any<kFmtGF4, false>(a, stream);
}

hipError_t launch_gf4_gemv_chunked(const GemvArgs& a, hipStream_t stream) {
    return a.w_up ? kq_gf4_swiglu(a, stream) : kq_gf4_plain(a, stream);
}

}  // namespace qw35
