// Chunked decode GEMV, q8_0, plain (and greedy-head) instantiations (kernel in kquant_mfma.h).
#include "kquant_mfma.h"

namespace qw35 {

hipError_t kq_q8_0_plain(const GemvArgs& a, hipStream_t stream) {
    return kq_launch_any<kFmtQ8, false>(a, stream);
}

hipError_t launch_q8_0_gemv(const GemvArgs& a, hipStream_t stream) {
    if (a.k % 256 != 0) return launch_q8_0_gemv_rows(a, stream);  // rows of 32-column blocks only
    return a.w_up ? kq_q8_0_swiglu(a, stream) : kq_q8_0_plain(a, stream);
}

}  // namespace qw35
