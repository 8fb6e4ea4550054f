// Host-only stand-ins for the kernel launchers of fa_params.hpp, for the
// sanitizer build of the C-ABI shim (csrc/fa_abi.cpp): every launcher records
// the parameter block it was given and returns success without touching a GPU.
#include "fa_params.hpp"
#include "stub_record.h"

StubRecord g_stub;

namespace fa {

#define STUB_FWD(name)                                                                       \
    hipError_t name(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t) {    \
        g_stub.fwd = p;                                                                      \
        g_stub.D = D;                                                                        \
        g_stub.causal = causal;                                                              \
        g_stub.dropout = dropout;                                                            \
        g_stub.fwd_calls++;                                                                  \
        g_stub.last = #name;                                                                 \
        return hipSuccess;                                                                   \
    }
#define STUB_BWD(name)                                                                                 \
    hipError_t name(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t) {    \
        g_stub.bwd = p;                                                                                \
        g_stub.D = D;                                                                                  \
        g_stub.causal = causal;                                                                        \
        g_stub.dropout = dropout;                                                                      \
        g_stub.stage = stage;                                                                          \
        g_stub.bwd_calls++;                                                                            \
        g_stub.last = #name;                                                                           \
        return hipSuccess;                                                                             \
    }

STUB_FWD(launch_fwd_bf16)
STUB_FWD(launch_fwd_f16)
STUB_FWD(launch_fwd_f32)
STUB_FWD(launch_fwd_bias_bf16)
STUB_FWD(launch_fwd_bias_f16)
STUB_FWD(launch_fwd_bias_f32)
STUB_FWD(launch_fwd_bias32_bf16)
STUB_FWD(launch_fwd_bias32_f16)
STUB_BWD(launch_bwd_bf16)
STUB_BWD(launch_bwd_f16)
STUB_BWD(launch_bwd_f32)
STUB_BWD(launch_bwd_bias_bf16)
STUB_BWD(launch_bwd_bias_f16)
STUB_BWD(launch_bwd_bias_f32)
STUB_BWD(launch_bwd_bias32_bf16)
STUB_BWD(launch_bwd_bias32_f16)
STUB_FWD(launch_fwd_d256_bf16)
STUB_FWD(launch_fwd_d256_f16)
STUB_BWD(launch_bwd_d256_bf16)
STUB_BWD(launch_bwd_d256_f16)

hipError_t launch_dropout_mask(uint64_t, uint64_t, int, int, int, int, float, uint8_t*, hipStream_t) {
    g_stub.misc_calls++;
    return hipSuccess;
}
hipError_t launch_rand(uint64_t, const uint64_t*, int64_t, float*, hipStream_t) {
    g_stub.misc_calls++;
    return hipSuccess;
}
hipError_t launch_keep_bits(const FwdParams&, bool, hipStream_t) {
    g_stub.keep_bits_calls++;
    return hipSuccess;
}
hipError_t launch_dbias_zero_tails(const BwdParams&, hipStream_t) {
    g_stub.misc_calls++;
    return hipSuccess;
}
hipError_t launch_dbias_reduce(const DbiasReduceParams& r, hipStream_t) {
    g_stub.reduce = r;
    g_stub.reduce_calls++;
    return hipSuccess;
}

}  // namespace fa
