// Backward kernel instantiations (delta pre-pass, dK/dV, dQ) for f16 inputs (D in
// {32, 64, 128}, causal x dropout), with an additive float32 bias.  One translation unit per pass,
// dtype and bias mode keeps builds parallel.
#include "fa_bwd.hpp"

namespace fa {

hipError_t launch_bwd_bias32_f16(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s) {
    return launch_bwd_dispatch<f16, float>(p, D, causal, dropout, stage, s);
}

}  // namespace fa
