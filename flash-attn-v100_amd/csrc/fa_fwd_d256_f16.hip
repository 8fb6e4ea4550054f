// Forward kernel instantiations for f16 inputs at head dim 256 (no bias), a
// translation unit of its own: its kernels hold up to 512 registers per lane
// and take the longest to compile.
#include "fa_fwd.hpp"

namespace fa {

hipError_t launch_fwd_d256_f16(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s) {
    if (D != 256) return hipErrorInvalidValue;
    return launch_fwd_d256<f16>(p, causal, dropout, s);
}

}  // namespace fa
