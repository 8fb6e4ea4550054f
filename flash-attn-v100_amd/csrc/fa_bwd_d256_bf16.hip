// Backward kernel instantiations for bf16 inputs at head dim 256 (no bias), a
// translation unit of its own: its kernels hold up to 512 registers per lane
// and take the longest to compile.
#include "fa_bwd.hpp"

namespace fa {

hipError_t launch_bwd_d256_bf16(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s) {
    if (D != 256) return hipErrorInvalidValue;
    return launch_bwd_d256<bf16>(p, causal, dropout, stage, s);
}

}  // namespace fa
