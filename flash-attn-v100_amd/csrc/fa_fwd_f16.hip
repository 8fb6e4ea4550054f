// Forward kernel instantiations for f16 inputs (D in {32, 64, 128}, causal x
// dropout), without a bias.  One translation unit per pass, dtype and bias
// mode keeps builds parallel.
#include "fa_fwd.hpp"

namespace fa {

hipError_t launch_fwd_f16(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s) {
    return launch_fwd_dispatch<f16, void>(p, D, causal, dropout, s);
}

}  // namespace fa
