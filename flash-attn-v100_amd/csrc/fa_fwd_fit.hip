// The causal copy-wave forward with slice groups sized to divide each XCD's
// slices (fwd_pp_kernel with FIT), for 16-bit inputs at D = 128.  Its own
// translation unit, so that the plain kernel compiles alone.
#include "fa_fwd.hpp"

namespace fa {

template <typename T>
hipError_t launch_fwd_pp_fit(const FwdParams& q, int64_t nblocks, hipStream_t s) {
    hipLaunchKernelGGL((fwd_pp_kernel<T, 128, true, true>), dim3((unsigned)nblocks), dim3(FwdPPCfg<T, 128>::NT), 0, s, q);
    return hipGetLastError();
}

template hipError_t launch_fwd_pp_fit<bf16>(const FwdParams&, int64_t, hipStream_t);
template hipError_t launch_fwd_pp_fit<f16>(const FwdParams&, int64_t, hipStream_t);

}  // namespace fa
