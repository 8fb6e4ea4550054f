// Test hooks exposing the device RNG exactly as the attention kernels use it,
// the forward's dropout keep bits, the broadcast reduction of the bias
// gradient and the zero tails of a causal bias gradient.
#include <algorithm>

#include "fa_abi.h"
#include "fa_common.hpp"
#include "fa_params.hpp"

namespace fa {

__global__ __launch_bounds__(256) void dropout_mask_kernel(uint64_t seed, uint64_t offset, int64_t n,
                                                           uint32_t thresh, uint8_t* __restrict__ keep) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) keep[i] = philox_keep(seed, offset + (uint64_t)i, thresh) ? 1 : 0;
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
    hipLaunchKernelGGL(dropout_mask_kernel, dim3((unsigned)nb), dim3(256), 0, s, seed, offset, n, keep_threshold(p),
                       keep);
    return hipGetLastError();
}

// Dropout keep bits: word w of row r = (b*H + h)*Sq + i holds keep(b, h, i,
// 32 w + t) at bit t.  A wave takes KB_ROWS consecutive rows and walks their
// keys 64 * KB_SETS at a time: lane l draws keys k0 + 64 v + l (v < KB_SETS)
// of each row (KB_ROWS * KB_SETS independent Philox chains, which hide each
// other's multiply latency), then one ballot per (row, v) gives two words,
// which lanes 0 and 1 store.  Under causal masking a group stops after the last
// key any of its queries sees (the bits of keys past a query's own diagonal
// are drawn but never read).  Rows (fewer than 2^31: B*H*Sq rows of q fit in
// memory) use 32-bit index math.
// 2 rows x 4 key groups: measured against 1 x 8, 4 x 2 and 8 x 1, the best
// balance between long rows (fewer groups per key) and short causal rows
// (less drawn past the diagonal)
constexpr int KB_ROWS = 2;
constexpr int KB_SETS = 8 / KB_ROWS;
__global__ __launch_bounds__(256) void keep_bits_kernel(uint64_t seed, uint64_t offset, uint32_t thresh,
                                                        uint32_t* __restrict__ kb, int kb_w, int Sq, int Sk, int rows,
                                                        int causal) {
    const int lane = threadIdx.x & 63;
    const int ngroups = (rows + KB_ROWS - 1) / KB_ROWS;
    const int step = gridDim.x * 4;
    for (int grp = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); grp < ngroups; grp += step) {
        const int r0 = grp * KB_ROWS;
        int kend = Sk;
        if (causal) {  // largest query index among the group's rows
            const int i0 = r0 % Sq, last = min(KB_ROWS, rows - r0) - 1;
            kend = min(Sk, (i0 + last < Sq ? i0 + last : Sq - 1) + 1);
        }
        for (int k0 = 0; k0 < kend; k0 += 64 * KB_SETS) {
            bool keep[KB_ROWS][KB_SETS];
#pragma unroll
            for (int u = 0; u < KB_ROWS; ++u)
#pragma unroll
                for (int v = 0; v < KB_SETS; ++v)
                    keep[u][v] = philox_keep(
                        seed, offset + (uint64_t)(r0 + u) * (uint64_t)Sk + (uint64_t)(k0 + 64 * v + lane), thresh);
#pragma unroll
            for (int u = 0; u < KB_ROWS; ++u)
#pragma unroll
                for (int v = 0; v < KB_SETS; ++v) {
                    // keys past Sk and rows past the last one draw too (never stored or read)
                    const uint64_t bal = __ballot(keep[u][v]);
                    const int w = ((k0 + 64 * v) >> 5) + lane;  // lanes 0, 1: the two 32-key words
                    if (lane < 2 && w < kb_w && r0 + u < rows)
                        kb[(int64_t)(r0 + u) * kb_w + w] = lane == 0 ? (uint32_t)bal : (uint32_t)(bal >> 32);
                }
        }
    }
}

hipError_t launch_keep_bits(const FwdParams& p, bool causal, hipStream_t s) {
    const int64_t rows = (int64_t)p.B * p.H * p.Sq;
    if (rows <= 0 || p.Sk <= 0) return hipSuccess;
    if (rows > 0x7fffffff - KB_ROWS) return hipErrorInvalidValue;
    const int64_t groups = (rows + KB_ROWS - 1) / KB_ROWS;
    const int64_t nb = std::min<int64_t>((groups + 3) / 4, 1 << 16);
    hipLaunchKernelGGL(keep_bits_kernel, dim3((unsigned)nb), dim3(256), 0, s, p.seed, p.offset, p.keep_thresh, p.kb,
                       p.kb_w, p.Sq, p.Sk, (int)rows, causal ? 1 : 0);
    return hipGetLastError();
}

// One thread per 16 bytes of part keys of one output row (KPT = 4 float32
// or 8 16-bit keys): one 16-byte load of every part slice that sums into it,
// summed in float32 in slice order (HBM-bound streaming, no atomics).  Part
// rows are whole 16-byte chunks (Sk rounded up); 16-bit parts have the output's
// dtype.
template <int KPT>
__global__ __launch_bounds__(256) void dbias_reduce_kernel(const DbiasReduceParams r) {
    const int njg = (r.Sk + KPT - 1) / KPT;
    const int Bo = r.sum_b ? 1 : r.B, Ho = r.sum_h ? 1 : r.H;
    const int64_t n = (int64_t)Bo * Ho * r.Sq * njg;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= n) return;
    const int j = (int)(t % njg) * KPT;
    int64_t rest = t / njg;
    const int i = (int)(rest % r.Sq);
    rest /= r.Sq;
    const int ho = (int)(rest % Ho), bo = (int)(rest / Ho);
    float acc[KPT];
    for (int e = 0; e < KPT; ++e) acc[e] = 0.f;
    if (!r.causal || j <= i) {
        const int b0 = r.sum_b ? 0 : bo, b1 = r.sum_b ? r.B : bo + 1;
        const int h0 = r.sum_h ? 0 : ho, h1 = r.sum_h ? r.H : ho + 1;
        for (int b = b0; b < b1; ++b)
            for (int h = h0; h < h1; ++h) {
                const int64_t pe = (((int64_t)b * r.H + h) * r.Sq + i) * r.SkP + j;  // element index
                const uint4 u = *reinterpret_cast<const uint4*>((const char*)r.part + pe * (16 / KPT));
                if constexpr (KPT == 4) {
                    const f32x4 v = __builtin_bit_cast(f32x4, u);
                    for (int e = 0; e < 4; ++e) acc[e] += v[e];
                } else {
                    const s16x8 v = __builtin_bit_cast(s16x8, u);
                    for (int e = 0; e < 8; ++e)
                        acc[e] += r.part_dtype == FA_DTYPE_BF16 ? Elem<bf16>::unpack1(v[e]) : Elem<f16>::unpack1(v[e]);
                }
            }
        if (r.causal)  // the part entries past the diagonal were never written
            for (int e = 1; e < KPT; ++e)
                if (j + e > i) acc[e] = 0.f;
    }
    const int64_t oe = bo * r.out_sb + ho * r.out_sh + (int64_t)i * r.out_ss + j;  // element index
    const int n_out = min(KPT, r.Sk - j);
    if (r.out_dtype == FA_DTYPE_F32) {
        float* o = (float*)r.out + oe;
        if (n_out == KPT)
            for (int e = 0; e < KPT; e += 4)
                *reinterpret_cast<float4*>(o + e) = make_float4(acc[e], acc[e + 1], acc[e + 2], acc[e + 3]);
        else
            for (int e = 0; e < n_out; ++e) o[e] = acc[e];
    } else {
        unsigned short h[KPT];
        for (int e = 0; e < KPT; ++e)
            h[e] = r.out_dtype == FA_DTYPE_BF16 ? __builtin_bit_cast(unsigned short, (bf16)acc[e])
                                                : __builtin_bit_cast(unsigned short, (f16)acc[e]);
        unsigned short* o = (unsigned short*)r.out + oe;
        if (n_out == KPT)  // 8-byte stores: the output's base and strides are multiples of 4 elements
            for (int e = 0; e < KPT; e += 4)
                *reinterpret_cast<uint2*>(o + e) =
                    make_uint2(h[e] | (unsigned)h[e + 1] << 16, h[e + 2] | (unsigned)h[e + 3] << 16);
        else
            for (int e = 0; e < n_out; ++e) o[e] = h[e];
    }
}

hipError_t launch_dbias_reduce(const DbiasReduceParams& r, hipStream_t s) {
    const int kpt = r.part_dtype == FA_DTYPE_F32 ? 4 : 8;
    const int64_t n = (int64_t)(r.sum_b ? 1 : r.B) * (r.sum_h ? 1 : r.H) * r.Sq * ((r.Sk + kpt - 1) / kpt);
    if (n <= 0) return hipSuccess;
    const int64_t nb = (n + 255) / 256;
    if (nb > 0x7fffffff) return hipErrorInvalidValue;
    if (kpt == 4)
        hipLaunchKernelGGL(dbias_reduce_kernel<4>, dim3((unsigned)nb), dim3(256), 0, s, r);
    else
        hipLaunchKernelGGL(dbias_reduce_kernel<8>, dim3((unsigned)nb), dim3(256), 0, s, r);
    return hipGetLastError();
}

// Causal gradient of a bias, written in place (dq_from_ds): the entries no
// kernel visits are keys from the end of each 128-query tile on (the dK/dV
// pass writes dS for keys below it, zeros included).  One workgroup per
// (batch, head, 128-query tile), a wave per row, 16-byte non-temporal stores
// (nothing reads these lines back); rows are whole 16-byte chunks (Sk * es and
// the strides are multiples of 16 bytes under dq_from_ds).  The same region as
// dq_ds_kernel's fill, so a caller may run this kernel beside the dK/dV pass:
// a small grid (a grid-stride loop over the tiles) and few registers, so that
// it fits beside the dK/dV workgroups instead of taking the CUs before them.
// Measured at B=4, H=32, S=4096 bf16 (bias and gradient (B, H, S, S)), fwd +
// bwd: 64 workgroups 3.52 ms, 128 3.53, 256 3.55, 32 3.64 (the zeros then
// outlast the backward); the tails written by the dQ pass instead, 3.62.
constexpr int kZeroTileRows = 128;
constexpr int kZeroMaxBlocks = 64;
__global__ __launch_bounds__(256) void dbias_zero_tails_kernel(const BwdParams p, const int n_qtiles, const int64_t n_tiles) {
    const int es = p.dbias_es;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int64_t t = blockIdx.x; t < n_tiles; t += gridDim.x) {
        const int qt = (int)(t % n_qtiles);  // longest tails first
        const int bh = (int)(t / n_qtiles);
        const int h = bh % p.H, b = bh / p.H;
        const int q0 = qt * kZeroTileRows;
        const int kz = q0 + kZeroTileRows;
        if (kz >= p.Sk) continue;
        const int nrow = min(kZeroTileRows, p.Sq - q0);
        const int cpr = (p.Sk - kz) * es / 16;
        char* zb = (char*)p.dbias + (b * p.dbias_sb + h * p.dbias_sh + (int64_t)q0 * p.dbias_ss + kz) * es;
        for (int r = w; r < nrow; r += 4)
            for (int c = lane; c < cpr; c += 64)
                __builtin_nontemporal_store(u32x4{0u, 0u, 0u, 0u},
                                            reinterpret_cast<u32x4*>(zb + (int64_t)r * p.dbias_ss * es + 16 * c));
    }
}

hipError_t launch_dbias_zero_tails(const BwdParams& p, hipStream_t s) {
    const int nq = (p.Sq + kZeroTileRows - 1) / kZeroTileRows;
    const int64_t nt = (int64_t)nq * p.H * p.B;
    if (nt <= 0) return hipSuccess;
    const int nb = (int)(nt < kZeroMaxBlocks ? nt : kZeroMaxBlocks);
    hipLaunchKernelGGL(dbias_zero_tails_kernel, dim3((unsigned)nb), dim3(256), 0, s, p, nq, nt);
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
