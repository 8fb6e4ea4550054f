// FlashAttention forward for gfx950 (reference: kernels/forward_kernel.py:18-243,
// with its normalisation, tail-mask, dropout-counter and LSE defects fixed).
//
// One workgroup = 4 waves = 128 queries of one (batch, head); wave w owns
// queries q0 + 32w .. q0 + 32w + 31, lane l owns query q0 + 32w + l%32.
// Scores are computed transposed, S^T = K Q^T, so the accumulator of lane l
// holds keys {8(r/4) + 4(l/32) + r%4} of ITS query: the softmax max/sum are
// lane-local plus one exchange with lane l^32, and the O^T = V^T P^T
// accumulator is lane-aligned with the softmax statistics (rescale is lane-local).
//   * Q lives in registers for the whole KV loop (MFMA B operand).
//   * K/V tiles stream through double-buffered LDS (one barrier per tile),
//     loaded with 16-byte global loads issued a full tile ahead.
//   * V is written to LDS transposed (V^T[d][slot(key)], key order permuted to
//     match the P accumulator layout), so PV operands are single ds_read_b128.
//   * exp2 with scale*log2(e) folded into one FMA; the running max is only
//     moved (and O rescaled) when it grows by more than 2^8, which is exact.
//   * causal: KV tiles past the last query are never loaded; tiles past a
//     wave's last query are skipped by that wave; only diagonal and tail tiles
//     run the masking variant of the tile step.
//   * fp32 inputs use v_mfma_f32_32x32x2_f32 with fp32 P.
#pragma once

#include <type_traits>

#include "fa_common.hpp"
#include "fa_params.hpp"

namespace fa {

template <typename T, int D>
struct FwdCfg {
    static constexpr bool F32 = Elem<T>::kF32;
    static constexpr int NW = 4;
    static constexpr int NT = 64 * NW;
    static constexpr int BM = 32 * NW;            // queries per workgroup
    static constexpr int BN = F32 ? 32 : 64;      // keys per tile
    static constexpr int NB = BN / 32;            // 32-key blocks per tile
    static constexpr int KW = D + (F32 ? 4 : 8);  // K row stride (elements)
    // V: fp32 keeps rows (stride D + 8); 16-bit types store V^T[d][slot(key)]
    static constexpr int VW = F32 ? D + 8 : BN + 8;
    static constexpr int KTILE = BN * KW;
    static constexpr int VTILE = F32 ? BN * VW : D * VW;
    static constexpr int OW = D + (F32 ? 4 : 8);  // output staging row stride
    static constexpr int SMEM_ELEMS = 2 * (KTILE + VTILE);
    static_assert(NW * 32 * OW <= SMEM_ELEMS, "O staging must fit in the K/V buffers");
};

template <typename T, int D, bool CAUSAL, bool DROPOUT>
__global__ __launch_bounds__(256, 2) void fwd_kernel(const FwdParams p) {
    using C = FwdCfg<T, D>;
    constexpr int BN = C::BN, NB = C::NB, KW = C::KW, VW = C::VW;
    __shared__ __attribute__((aligned(16))) T smem[C::SMEM_ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, l32 = lane & 31, hi = lane >> 5;

    const int L = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = L / p.n_qtiles;
    const int qt = p.n_qtiles - 1 - (L - bh * p.n_qtiles);  // longest causal rows first
    const int h = bh % p.H, b = bh / p.H;
    const int hk = h / p.group;
    const int q0 = qt * C::BM;
    const int qw0 = q0 + 32 * w;
    const int qi = qw0 + l32;

    const T* __restrict__ kbase = (const T*)p.k + b * p.k_sb + hk * p.k_sh;
    const T* __restrict__ vbase = (const T*)p.v + b * p.v_sb + hk * p.v_sh;

    int kv_end = p.Sk;
    if (CAUSAL) kv_end = min(kv_end, min(q0 + C::BM, p.Sq));
    const int n_tiles = (kv_end + BN - 1) / BN;
    // tiles before n_plain need no masking for any wave of the workgroup
    int n_plain = min(n_tiles, p.Sk / BN);
    if (CAUSAL) n_plain = min(n_plain, (q0 + 1) / BN);

    // ---- Q into registers (MFMA B operand) ----
    constexpr int QR = C::F32 ? D / 8 : D / 16;  // 16-byte registers per lane
    uint4 qreg[QR];
    {
        const T* qrow = (const T*)p.q + b * p.q_sb + (int64_t)qi * p.q_ss + h * p.q_sh;
#pragma unroll
        for (int i = 0; i < QR; ++i) {
            // bf16/f16: d = 16i + 8hi .. +7 ; f32: d = hi*D/2 + 4i .. +3
            const int d0 = C::F32 ? hi * (D / 2) + 4 * i : 16 * i + 8 * hi;
            qreg[i] = qi < p.Sq ? *reinterpret_cast<const uint4*>(qrow + d0) : make_uint4(0u, 0u, 0u, 0u);
        }
    }
    wait_vmem();

    f32x16 o[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) o[i] = f32x16{};
    float m_run = -1e30f;  // running max in log2 units (scores * scale * log2 e)
    float l_run = 0.f;     // lane-partial row sum of exp2(t - m_run)
    float m_raw = -INFINITY;
    const float c = p.scale_log2;

    uint64_t row_ctr = 0;
    if (DROPOUT) row_ctr = p.offset + ((uint64_t)(b * p.H + h) * (uint64_t)p.Sq + (uint64_t)qi) * (uint64_t)p.Sk;

    T* Ks0 = smem;
    T* Vs0 = smem + 2 * C::KTILE;
    using KStage = typename std::conditional<C::F32, TileStage<T, BN, D, C::NT>, Tile16<T, BN, D, C::NT>>::type;
    KStage kst, vst;
    auto load_tile = [&](int k0) {
        kst.load(kbase + (int64_t)k0 * p.k_ss, p.k_ss, p.Sk - k0, tid);
        vst.load(vbase + (int64_t)k0 * p.v_ss, p.v_ss, p.Sk - k0, tid);
    };
    auto store_tile = [&](int buf) {
        if constexpr (C::F32) {
            kst.template store<KW>(Ks0 + buf * C::KTILE, tid);
            vst.template store<VW>(Vs0 + buf * C::VTILE, tid);
        } else {
            kst.template store_rows<KW>(Ks0 + buf * C::KTILE, tid);
            vst.template store_trans<VW>(Vs0 + buf * C::VTILE, tid);
        }
    };

    // one KV tile; MASK selects the diagonal/tail variant
    auto step = [&](int j, auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int k0 = j * BN;
        if (j + 1 < n_tiles) load_tile(k0 + BN);
        lds_barrier();
        const T* Ks = Ks0 + (j & 1) * C::KTILE;
        const T* Vs = Vs0 + (j & 1) * C::VTILE;

        const bool active = !MASK || !CAUSAL || k0 <= qw0 + 31;
        if (active) {
            // ---- S^T = K Q^T ----
            f32x16 s[NB];
#pragma unroll
            for (int blk = 0; blk < NB; ++blk) {
                s[blk] = f32x16{};
                const T* krow = Ks + (32 * blk + l32) * KW;
                if constexpr (C::F32) {
#pragma unroll
                    for (int i = 0; i < QR; ++i) {
                        const f32x4 a = *reinterpret_cast<const f32x4*>(krow + hi * (D / 2) + 4 * i);
                        const f32x4 bq = __builtin_bit_cast(f32x4, qreg[i]);
#pragma unroll
                        for (int e = 0; e < 4; ++e) s[blk] = mfma_f32(a[e], bq[e], s[blk]);
                    }
                } else {
#pragma unroll
                    for (int kk = 0; kk < QR; ++kk) {
                        const s16x8 a = *reinterpret_cast<const s16x8*>(krow + 16 * kk + 8 * hi);
                        s[blk] = Elem<T>::mfma(a, __builtin_bit_cast(s16x8, qreg[kk]), s[blk]);
                    }
                }
            }
            if constexpr (MASK) {
                const bool need = (k0 + BN > p.Sk) || (CAUSAL && k0 + BN - 1 > qw0);
                if (need) {
#pragma unroll
                    for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int key = k0 + 32 * blk + 8 * (r >> 2) + 4 * hi + (r & 3);
                            if (key >= p.Sk || (CAUSAL && key > qi)) s[blk][r] = -INFINITY;
                        }
                }
            }
            // ---- online softmax ----
            float mx = -INFINITY;
#pragma unroll
            for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[blk][r]);
            mx = fmaxf(mx, swap_halves(mx));
            m_raw = fmaxf(m_raw, mx);
            const float m_new = fmaxf(m_run, mx * c);
            if (__ballot(m_new > m_run + 8.0f) != 0ull) {
                const float alpha = fast_exp2(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int i = 0; i < D / 32; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
                m_run = m_new;
            }
            float psum = 0.f;
#pragma unroll
            for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float pv = fast_exp2(__builtin_fmaf(s[blk][r], c, -m_run));
                    psum += pv;
                    s[blk][r] = pv;
                }
            l_run += psum;
            if (DROPOUT) {
#pragma unroll
                for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = k0 + 32 * blk + 8 * (r >> 2) + 4 * hi + (r & 3);
                        const float u = philox_uniform(p.seed, row_ctr + (uint64_t)key);
                        if (!(u > p.dropout_p)) s[blk][r] = 0.f;
                    }
            }
            // ---- O^T += V^T P^T ----
            if constexpr (C::F32) {
#pragma unroll
                for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                    for (int t = 0; t < 16; ++t) {
                        const T* vrow = Vs + (32 * blk + 8 * (t >> 2) + 4 * hi + (t & 3)) * VW + l32;
#pragma unroll
                        for (int i = 0; i < D / 32; ++i) o[i] = mfma_f32(vrow[32 * i], s[blk][t], o[i]);
                    }
            } else {
#pragma unroll
                for (int ks = 0; ks < BN / 16; ++ks) {
                    float tmp[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) tmp[e] = s[ks >> 1][8 * (ks & 1) + e];
                    const s16x8 pk = pack8<T>(tmp);
#pragma unroll
                    for (int i = 0; i < D / 32; ++i) {
                        const s16x8 a = *reinterpret_cast<const s16x8*>(Vs + (32 * i + l32) * VW + 16 * ks + 8 * hi);
                        o[i] = Elem<T>::mfma(a, pk, o[i]);
                    }
                }
            }
        }
        if (j + 1 < n_tiles) store_tile((j + 1) & 1);
    };

    if (n_tiles > 0) {
        load_tile(0);
        store_tile(0);
    }
    for (int j = 0; j < n_plain; ++j) step(j, std::false_type{});
    for (int j = n_plain; j < n_tiles; ++j) step(j, std::true_type{});

    // ---- epilogue: normalise, LSE, stage O^T through LDS, coalesced store ----
    const float l_tot = l_run + swap_halves(l_run);
    const float inv = l_tot > 0.f ? (DROPOUT ? p.rp : 1.f) / l_tot : 0.f;
    if (hi == 0 && qi < p.Sq) {
        const int64_t si = (int64_t)(b * p.H + h) * p.Sq + qi;
        p.lse[si] = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
        if (p.mx) p.mx[si] = m_raw * p.scale;
    }
    lds_barrier();  // all waves done with the K/V buffers
    constexpr int OW = C::OW;
    T* Os = smem + w * 32 * OW;
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * i + 8 * g + 4 * hi;
            if constexpr (C::F32) {
                f32x4 v4;
#pragma unroll
                for (int e = 0; e < 4; ++e) v4[e] = o[i][4 * g + e] * inv;
                *reinterpret_cast<f32x4*>(Os + l32 * OW + d) = v4;
            } else {
                s16x4 v4;
#pragma unroll
                for (int e = 0; e < 4; ++e) v4[e] = Elem<T>::pack1(o[i][4 * g + e] * inv);
                *reinterpret_cast<s16x4*>(Os + l32 * OW + d) = v4;
            }
        }
    lds_barrier();
    constexpr int EPC = 16 / sizeof(T);
    constexpr int CPR = D / EPC;
    T* obase = (T*)p.o + b * p.o_sb + h * p.o_sh;
#pragma unroll
    for (int i = 0; i < 32 * CPR / 64; ++i) {
        const int cidx = lane + 64 * i;
        const int row = cidx / CPR, col = cidx % CPR;
        const int q = qw0 + row;
        if (q < p.Sq)
            *reinterpret_cast<uint4*>(obase + (int64_t)q * p.o_ss + col * EPC) =
                *reinterpret_cast<const uint4*>(Os + row * OW + col * EPC);
    }
}

template <typename T, int D, bool CAUSAL, bool DROPOUT>
hipError_t launch_fwd_t(const FwdParams& p, hipStream_t s) {
    using C = FwdCfg<T, D>;
    FwdParams q = p;
    q.n_qtiles = (p.Sq + C::BM - 1) / C::BM;
    const int64_t nblocks = (int64_t)q.n_qtiles * p.H * p.B;
    if (nblocks <= 0) return hipSuccess;
    hipLaunchKernelGGL((fwd_kernel<T, D, CAUSAL, DROPOUT>), dim3((unsigned)nblocks), dim3(C::NT), 0, s, q);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_fwd_dispatch(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s) {
#define FA_FWD_CASE(DD)                                                                  \
    if (D == DD) {                                                                       \
        if (causal) return dropout ? launch_fwd_t<T, DD, true, true>(p, s)               \
                                   : launch_fwd_t<T, DD, true, false>(p, s);             \
        return dropout ? launch_fwd_t<T, DD, false, true>(p, s)                          \
                       : launch_fwd_t<T, DD, false, false>(p, s);                        \
    }
    FA_FWD_CASE(32)
    FA_FWD_CASE(64)
    FA_FWD_CASE(128)
#undef FA_FWD_CASE
    return hipErrorInvalidValue;
}

}  // namespace fa
