// Forward kernel instantiations for f32 inputs (D in {32, 64, 128}, causal x
// dropout), with an additive bias of the input dtype.  One translation unit per pass, dtype and bias
// mode keeps builds parallel.
#include "fa_fwd.hpp"

namespace fa {

hipError_t launch_fwd_bias_f32(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s) {
    return launch_fwd_dispatch<float, float>(p, D, causal, dropout, s);
}

}  // namespace fa
