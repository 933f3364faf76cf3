// Prefill-path (m > 8) int8 MFMA kernels.  Placeholder until the MFMA path
// lands: reports no support, so matmul routes every m through the matvec.
#include "xnq_internal.h"

namespace xnq {

bool mfma_supported(uint32_t, size_t, size_t, size_t) { return false; }

hipError_t launch_mfma(const WView&, const AView&, size_t, float*, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace xnq
