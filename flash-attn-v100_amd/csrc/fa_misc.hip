// Test hooks exposing the device RNG exactly as the attention kernels use it.
#include "fa_common.hpp"
#include "fa_params.hpp"

namespace fa {

__global__ __launch_bounds__(256) void dropout_mask_kernel(uint64_t seed, uint64_t offset, int64_t n,
                                                           float p, uint8_t* __restrict__ keep) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) keep[i] = philox_uniform(seed, offset + (uint64_t)i) > p ? 1 : 0;
}

__global__ __launch_bounds__(256) void rand_kernel(uint64_t seed, const uint64_t* __restrict__ ctr, int64_t n,
                                                   float* __restrict__ u) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) u[i] = philox_uniform(seed, ctr[i]);
}

// The (B, H, Sq, Sk) element index is exactly ((b*H + h)*Sq + i)*Sk + j, so
// the dropout counter of element e is offset + e.
hipError_t launch_dropout_mask(uint64_t seed, uint64_t offset, int B, int H, int Sq, int Sk, float p,
                               uint8_t* keep, hipStream_t s) {
    const int64_t n = (int64_t)B * H * Sq * Sk;
    if (n <= 0) return hipSuccess;
    const int64_t nb = (n + 255) / 256;
    if (nb > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dropout_mask_kernel, dim3((unsigned)nb), dim3(256), 0, s, seed, offset, n, p, keep);
    return hipGetLastError();
}

hipError_t launch_rand(uint64_t seed, const uint64_t* ctr, int64_t n, float* u, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t nb = (n + 255) / 256;
    if (nb > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rand_kernel, dim3((unsigned)nb), dim3(256), 0, s, seed, ctr, n, u);
    return hipGetLastError();
}

}  // namespace fa
