// Forward and backward kernel instantiations for f32 inputs (D in {32, 64, 128},
// causal x dropout), without a bias.  One translation unit per dtype and bias mode
// keeps builds parallel.
#include "fa_bwd.hpp"
#include "fa_fwd.hpp"

namespace fa {

hipError_t launch_fwd_f32(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s) {
    return launch_fwd_dispatch<float, void>(p, D, causal, dropout, s);
}

hipError_t launch_bwd_f32(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s) {
    return launch_bwd_dispatch<float, void>(p, D, causal, dropout, stage, s);
}

}  // namespace fa
