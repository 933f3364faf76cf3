// Matvec kernels for XNQ_Q4_1 weights (instantiations of k_matvec_impl.h).
#include "k_matvec_impl.h"

namespace xnq {

hipError_t launch_matvec_q4_1(const WView& w, const AView& a, const float* x, size_t m, float* y, hipStream_t s,
                            int fused) {
    return mv::launch_dtype<XNQ_Q4_1>(w, a, x, m, y, s, fused);
}

hipError_t launch_group_q4_1(const WGroup& g, const float* x, bool gate, hipStream_t s) {
    return launch_group_dt<XNQ_Q4_1>(g, x, gate, s);
}

}  // namespace xnq
