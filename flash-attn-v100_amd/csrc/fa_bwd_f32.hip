// Backward kernel instantiations (delta pre-pass, dK/dV, dQ) for f32 inputs (D in
// {32, 64, 128}, causal x dropout), without a bias.  One translation unit per pass,
// dtype and bias mode keeps builds parallel.
#include "fa_bwd.hpp"

namespace fa {

hipError_t launch_bwd_f32(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s) {
    return launch_bwd_dispatch<float, void>(p, D, causal, dropout, stage, s);
}

}  // namespace fa
