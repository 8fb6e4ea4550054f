// FlashAttention backward for gfx950 (reference: kernels/backward_kernel.py:17-205,
// whose racy low-precision dQ read-modify-write and per-tile-pair delta are
// replaced).  Three deterministic kernels, no atomics:
//   1. delta_kernel: LSE * log2 e and delta = rowsum(dO * O) in fp32 into the
//      workspace rows.
//   2. dkdv_kernel: one workgroup per 128 keys of one (batch, KV head); wave w
//      owns keys k0 + 32w .. +31 (lane l owns key k0 + 32w + l%32), K and V rows
//      stay in registers; 64-query tiles of Q, dO and the LSE / delta rows are
//      copied global -> LDS (double-buffered) and consumed as two 32-query
//      sub-steps.  Scores are computed as S = Q K^T so each lane holds queries
//      {8(r/4) + 4(l/32) + r%4} of ITS key, which is exactly the MFMA
//      B-operand layout needed for dV^T = dO^T P and dK^T = Q^T dS (the dO^T /
//      Q^T operands come from the row-major LDS tiles via ds_read_b64_tr_b16).
//      Query heads sharing a KV head are summed in-register.
//   3. dq_kernel: one workgroup per 128 queries of one (batch, head), like the
//      forward: S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T with Q, dO, LSE,
//      delta held per lane; 64-key K/V tiles are copied global -> LDS
//      (double-buffered) and consumed as two 32-key sub-steps, K^T read from
//      the K tile with transposing reads.
// Variants of the same arithmetic: dkdv8_kernel (K and V in LDS, 8 waves: small
// grids and a bias), dkdv_pp_kernel / dq_pp_kernel (8-wave ping-pong workgroups
// of 256 keys / queries: 16-bit D = 128 grids that fill the chip),
// bwd_small_kernel (the dK/dV and dQ workgroups of a small grid in one launch),
// dq_ds_kernel (dQ from the dS a bias-gradient pass stored).
// Diagonal (causal) tiles run a separate masking variant of each tile step.
// With an additive bias (BIAS) both kernels add bias * log2 e to the scores
// before the exponent; dkdv_kernel, the one kernel that visits every
// (query, key) pair once, also writes dBias = dS (unscaled, rounded once to the
// requested dtype) when asked.
// All five products accumulate in fp32 and are rounded once to the input dtype.
#pragma once

#include <type_traits>

#include "fa_common.hpp"
#include "fa_params.hpp"

namespace fa {

// ---------------------------------------------------------------------------
// delta = rowsum(dO * O) and LSE * log2(e) into the padded workspace rows;
// padding rows (Sq <= i < sq_pad) get delta = 0 and LSE * log2(e) = +inf, so
// a query tile that reads them gets P = 0 without a range check; so do rows
// whose saved LSE is -inf.
template <typename T, int D>
__global__ __launch_bounds__(256) void delta_kernel(const BwdParams p) {
    constexpr int EPC = 16 / sizeof(T);
    constexpr int LPR = D / EPC;        // lanes per row
    constexpr int RPB = 256 / LPR;      // rows per block
    const int tid = threadIdx.x;
    const int64_t row = (int64_t)blockIdx.x * RPB + tid / LPR;
    const int part = tid % LPR;
    const int64_t nrows = (int64_t)p.B * p.sq_pad * p.H;
    float acc = 0.f;
    int b = 0, i = 0, h = 0;
    if (row < nrows) {
        h = (int)(row % p.H);
        const int64_t bi = row / p.H;
        i = (int)(bi % p.sq_pad);
        b = (int)(bi / p.sq_pad);
    }
    if (row < nrows && i < p.Sq) {
        const T* orow = (const T*)p.o + b * p.o_sb + (int64_t)i * p.o_ss + h * p.o_sh + part * EPC;
        const T* drow = (const T*)p.dout + b * p.do_sb + (int64_t)i * p.do_ss + h * p.do_sh + part * EPC;
        const uint4 ov = *reinterpret_cast<const uint4*>(orow);
        const uint4 dv = *reinterpret_cast<const uint4*>(drow);
        if constexpr (Elem<T>::kF32) {
            const f32x4 a = __builtin_bit_cast(f32x4, ov), c = __builtin_bit_cast(f32x4, dv);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc += a[e] * c[e];
        } else {
            const s16x8 a = __builtin_bit_cast(s16x8, ov), c = __builtin_bit_cast(s16x8, dv);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc += Elem<T>::unpack1(a[e]) * Elem<T>::unpack1(c[e]);
        }
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (row < nrows && part == 0) {
        const int64_t wi = ((int64_t)b * p.H + h) * p.ws_stride + i;
        p.delta[wi] = acc;
        // a row with no visible key (every score -inf, e.g. a fully masked bias
        // row) has LSE = -inf and O = 0: +inf here makes its P = 0, so its
        // gradients are 0 instead of NaN
        const float l = i < p.Sq ? p.lse[((int64_t)b * p.H + h) * p.Sq + i] : -INFINITY;
        p.lse2[wi] = l == -INFINITY ? INFINITY : l * kLog2e;
    }
}

// ---------------------------------------------------------------------------
// -x for eight 16-bit floats (the sign bits)
__device__ FA_INLINE inline uint4 neg16x8(uint4 v) {
    v.x ^= 0x80008000u;
    v.y ^= 0x80008000u;
    v.z ^= 0x80008000u;
    v.w ^= 0x80008000u;
    return v;
}
// delta of the 16 queries {8 g + 4 hi + e} of a 32-query sub-step in the
// accumulator order of a lane (a key per lane), from the sub-step's LDS row
__device__ FA_INLINE inline f32x16 delta16(const float* d, int hi) {
    f32x16 r;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(d + 8 * g + 4 * hi);
#pragma unroll
        for (int e = 0; e < 4; ++e) r[4 * g + e] = d4[e];
    }
    return r;
}

// ---------------------------------------------------------------------------
template <typename T, int D>
struct DkdvCfg {
    static constexpr bool F32 = Elem<T>::kF32;
    static constexpr int NW = 4;
    static constexpr int NT = 64 * NW;
    static constexpr int BK = 32 * NW;              // keys per workgroup
    static constexpr int NSUB = 2;                  // 32-query sub-tiles per tile
    static constexpr int BQ = 32 * NSUB;            // queries per tile
    // Q / dO row stride: odd multiple of 16 bytes (conflict-free ds_read_b128
    // row reads) whose 4 consecutive rows of a ds_read_b64_tr_b16 do not overlap
    // in the 256-byte bank window
    static constexpr int RW = D + (F32 ? 4 : (D == 64 ? 8 : 24));
    static constexpr int QTILE = BQ * RW;
    // Q (waves 0-1) and dO (waves 2-3) tiles are copied global -> LDS directly
    using Rows = DmaRowGroups<T, BQ, D, RW, NW / 2>;
    static constexpr int QALLOC = BQ * RW * (int)sizeof(T);
    // per buffer: Q rows, dO rows, then LSE * log2 e [BQ] and delta [BQ] as floats
    static constexpr int BUF_BYTES = 2 * QALLOC + 2 * BQ * 4;
    static constexpr int NBUF = 2;                  // tile t read while t+1 lands
    static constexpr int OW = D + (F32 ? 4 : 8);    // output staging stride
    static constexpr int SMEM_BYTES_RAW = NBUF * BUF_BYTES;
    static constexpr int STAGE_BYTES = NW * 32 * OW * (int)sizeof(T);
    static constexpr int SMEM_BYTES = SMEM_BYTES_RAW > STAGE_BYTES ? SMEM_BYTES_RAW : STAGE_BYTES;
    static_assert(BUF_BYTES % 16 == 0, "16-byte aligned buffers");
};

// TB: element type of the additive bias (T or float), void = no bias.
// DA, DOFF: the kernel accumulates (and writes) only the dK / dV columns
// [DOFF, DOFF + DA); S and dP still take every column of Q, K, V and dO.  Head
// dim 256 runs it as two launches of 128 columns each: the dK / dV
// accumulators of all 256 columns (256 floats a lane) beside the K and V rows
// (128 registers) do not fit the 512 registers of a lane, and spilled them
// (about 1.1 KiB of scratch a lane); the halves recompute S and dP, 1.5x the
// products of one launch, with nothing spilled.
template <typename T, int D, bool CAUSAL, int DROPOUT, typename TB, int DA = D, int DOFF = 0>
__global__ __launch_bounds__(256, ((std::is_void<TB>::value || D <= 64) && !(Elem<T>::kF32 && D == 128) && D <= 128 ? 2 : 1)) void dkdv_kernel(
    const BwdParams p, const int n_ktiles) {
    using C = DkdvCfg<T, D>;
    static_assert(DA % 32 == 0 && DOFF % 32 == 0 && DOFF + DA <= D, "a range of whole 32-column blocks");
    constexpr bool BIAS = !std::is_void<TB>::value;
    using BT = typename std::conditional<BIAS, TB, T>::type;
    constexpr int BQ = C::BQ, RW = C::RW;
    // 16-bit inputs without bias or dropout: the dP products start from delta
    // and take -V, so they give delta - dP, and dS = P (dP - delta) costs one
    // product a score; the products then sum -dS into dK (-scale at the end).
    // (dkdv_pp_kernel does the same, bit for bit.)
    constexpr bool DFOLD = !C::F32 && !BIAS && DROPOUT == 0;
    __shared__ __attribute__((aligned(16))) char smem[C::SMEM_BYTES];

    const int tid = threadIdx.x;
    // wave index as a scalar: loop bounds derived from it stay wave-uniform
    const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), l32 = lane & 31, hi = lane >> 5;
    // key block kt = 0 sees the most queries (causal): rank order is kt order
    const int2 tord = tile_order<32 * ((std::is_void<TB>::value || D <= 64) && !(Elem<T>::kF32 && D == 128) && D <= 128 ? 2 : 1), CAUSAL>(n_ktiles);
    const int kt = tord.y;
    const int2 sbh = slice_bh(tord.x, p.Hkv, p.B, !std::is_void<TB>::value && p.bias_sb == 0);
    const int hk = sbh.y, b = sbh.x;
    const int k0 = kt * C::BK;
    const int kw0 = k0 + 32 * w;
    const int kj = kw0 + l32;  // this lane's key

    // ---- K, V rows of this lane's key in registers (MFMA B operands) ----
    constexpr int KR = C::F32 ? D / 8 : D / 16;
    uint4 kreg[KR], vreg[KR];
    {
        const T* krow = (const T*)p.k + b * p.k_sb + (int64_t)kj * p.k_ss + hk * p.k_sh;
        const T* vrow = (const T*)p.v + b * p.v_sb + (int64_t)kj * p.v_ss + hk * p.v_sh;
#pragma unroll
        for (int i = 0; i < KR; ++i) {
            const int d0 = C::F32 ? hi * (D / 2) + 4 * i : 16 * i + 8 * hi;
            const bool ok = kj < p.Sk;
            kreg[i] = ok ? *reinterpret_cast<const uint4*>(krow + d0) : make_uint4(0u, 0u, 0u, 0u);
            vreg[i] = ok ? *reinterpret_cast<const uint4*>(vrow + d0) : make_uint4(0u, 0u, 0u, 0u);
        }
        if constexpr (DFOLD) {
#pragma unroll
            for (int i = 0; i < KR; ++i) vreg[i] = neg16x8(vreg[i]);
        }
    }
    // no wait here: the K / V loads stay in flight while the first tile copy
    // is issued (the loop's first barrier waits for both)

    f32x16 dk[DA / 32], dv[DA / 32];
#pragma unroll
    for (int i = 0; i < DA / 32; ++i) { dk[i] = f32x16{}; dv[i] = f32x16{}; }
    const float c = p.scale_log2;

    // query tiles: causal needs queries >= k0 only; per query head of the
    // group the tiles run from the last one down, so that all workgroups of a
    // head read the same Q / dO tiles at about the same time (L2 reuse), and
    // the final tiles of the run cross this wave's keys and are masked
    const int qt_begin = CAUSAL ? (k0 / BQ) : 0;
    const int qt_end = (p.Sq + BQ - 1) / BQ;
    const int nq = qt_end > qt_begin ? qt_end - qt_begin : 0;
    const int total = nq * p.group;  // (head in group) x (query tile)
    const int n_mask = CAUSAL ? min(nq, max(0, (kw0 + 31 + BQ - 1) / BQ - qt_begin)) : 0;

    // ---- tiles: Q, dO rows and the LSE / delta rows, global -> LDS directly ----
    // waves 0-1 copy Q, waves 2-3 copy dO (scalar selects, no branches); every
    // wave copies the tile's LSE * log2 e and delta (one dword per lane, the
    // same values), so a tile copy is branch-free and can sit between MFMAs
    const bool copy_q = w < C::NW / 2;
    typename C::Rows rows;
    rows.init(copy_q ? p.q_ss : p.do_ss, lane, w % (C::NW / 2));
    static_assert(BQ == 64, "one dword per lane for each of LSE and delta");
    auto buf = [&](int s) -> char* { return smem + s * C::BUF_BYTES; };
    auto tile_head = [&](int it) { return hk * p.group + it / nq; };
    auto tile_q0 = [&](int it) { return (qt_end - 1 - it % nq) * BQ; };
    auto issue = [&](int it, int s) FA_INLINE {
        const int hh = tile_head(it), qb0 = tile_q0(it);
        char* bp = buf(s);
        const T* src = copy_q ? (const T*)p.q + b * p.q_sb + (int64_t)qb0 * p.q_ss + hh * p.q_sh
                              : (const T*)p.dout + b * p.do_sb + (int64_t)qb0 * p.do_ss + hh * p.do_sh;
        // copies the compiler does not track: it would otherwise make the
        // next LDS read of the current tile wait for them (sync_tiles waits)
        rows.load_untracked(src, copy_q ? p.q_ss : p.do_ss, p.Sq - qb0, (const T*)(bp + (copy_q ? 0 : C::QALLOC)));
        const float* wrow = p.lse2 + ((int64_t)b * p.H + hh) * p.ws_stride + qb0;  // qb0 + BQ <= sq_pad
        const u32x4 rs = buffer_words(wrow, (p.ws_stride - qb0) * 4);
        const uint32_t f = lds_addr(bp + 2 * C::QALLOC);
        dma_load4_untracked(rs, f, 4 * lane);                       // LSE * log2 e
        dma_load4_untracked(rs, f + 4 * BQ, 4 * (p.sq_pad + lane));  // delta
    };
    // direct-to-LDS copies complete when the issuing wave's vmcnt drains
    auto sync_tiles = [&]() {
        wait_vmem();
        lds_barrier();
    };

    // ---- S = Q K^T and dP = dO V^T for the tile in buffer s (C[q][key]) ----
    auto sdp = [&](int s, int st, f32x16& sc, f32x16& dpc) FA_INLINE {
        const T* Qs = (const T*)buf(s);
        const T* Ds = (const T*)(buf(s) + C::QALLOC);
        sc = f32x16{};
        if constexpr (DFOLD)
            dpc = delta16((const float*)(buf(s) + 2 * C::QALLOC) + BQ + 32 * st, hi);
        else
            dpc = f32x16{};
        const T* qrow = Qs + (32 * st + l32) * RW;
        const T* drow = Ds + (32 * st + l32) * RW;
        if constexpr (C::F32) {
#pragma unroll
            for (int i = 0; i < KR; ++i) {
                const f32x4 aq = *reinterpret_cast<const f32x4*>(qrow + hi * (D / 2) + 4 * i);
                const f32x4 ad = *reinterpret_cast<const f32x4*>(drow + hi * (D / 2) + 4 * i);
                const f32x4 bk = __builtin_bit_cast(f32x4, kreg[i]);
                const f32x4 bv = __builtin_bit_cast(f32x4, vreg[i]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sc = mfma_f32(aq[e], bk[e], sc);
                    dpc = mfma_f32(ad[e], bv[e], dpc);
                }
            }
        } else {
#pragma unroll
            for (int kk = 0; kk < KR; ++kk) {
                const s16x8 aq = *reinterpret_cast<const s16x8*>(qrow + 16 * kk + 8 * hi);
                const s16x8 ad = *reinterpret_cast<const s16x8*>(drow + 16 * kk + 8 * hi);
                sc = Elem<T>::mfma(aq, __builtin_bit_cast(s16x8, kreg[kk]), sc);
                dpc = Elem<T>::mfma(ad, __builtin_bit_cast(s16x8, vreg[kk]), dpc);
            }
        }
    };

    // ---- bias of this lane's key for the 16 queries {8 g + 4 hi + e} of a sub-step ----
    // one per-lane offset (key, row parity); the query rows go in the scalar
    // offset.  Rows past Sq read zeros (P = 0 there anyway); lanes past Sk read
    // zeros or another row and are never stored.
    // 16-bit values are kept two to a register (rows r, r + 1).  The values of
    // the next sub-step are loaded while the current one computes (bnext).
    constexpr bool B16 = BIAS && !Elem<BT>::kF32;
    constexpr int NBI = BIAS ? (B16 ? 8 : 16) : 1;
    using BR = typename std::conditional<B16, s16x2, float>::type;
    BR braw[NBI], bnext[NBI];
    const int bvoff = (4 * hi * (int)p.bias_ss + kj) * (int)sizeof(BT);
    auto load_bias = [&](BR (&dst)[NBI], int it, int st) FA_INLINE {
        if constexpr (BIAS) {
            const __amdgpu_buffer_rsrc_t rs =
                slice_buffer((const BT*)p.bias + b * p.bias_sb + tile_head(it) * p.bias_sh, p.bias_span);
            const int qb0 = tile_q0(it) + 32 * st;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const auto x = load_bias1<BT>(rs, bvoff, (qb0 + 8 * (r >> 2) + (r & 3)) * (int)p.bias_ss * (int)sizeof(BT));
                if constexpr (B16)
                    dst[r >> 1][r & 1] = x;
                else
                    dst[r] = x;
            }
        }
    };
    auto bias_at = [&](int r) FA_INLINE {
        if constexpr (B16)
            return braw[r >> 1][r & 1];
        else
            return braw[r];
    };
    // dBias stores: lanes past Sk are sent out of range; rows past Sq land past
    // the slice (query stride >= Sk) and are dropped
    const int dbvoff = kj < p.Sk ? (4 * hi * (int)p.dbias_ss + kj) * p.dbias_es : kOffNowhere;
    auto dbias_buf = [&](int hh) FA_INLINE {
        return slice_buffer((const char*)p.dbias + (b * p.dbias_sb + hh * p.dbias_sh) * p.dbias_es, p.dbias_span);
    };

    // ---- P and dS of tile `it` (buffer s); dS = P (dP - delta), scale applied at the end ----
    constexpr int NPK = C::F32 ? 1 : 2;
    float pd[16], ds[16];
    s16x8 bp8[NPK], bs8[NPK];
    auto softmax_ds = [&](int it, int s, int st, const f32x16& sc, const f32x16& dpc, uint32_t kword,
                          auto mask_tag) FA_INLINE {
        constexpr bool MASK = decltype(mask_tag)::value;
        const float* lse2 = (const float*)(buf(s) + 2 * C::QALLOC) + 32 * st;
        const float* dels = lse2 + BQ;
        const int qb0 = tile_q0(it) + 32 * st;
        const bool want_db = BIAS && p.dbias != nullptr;
        const __amdgpu_buffer_rsrc_t dbrs = dbias_buf(tile_head(it));
        // dropout keep of query q: the Philox stream regenerated (mode 1), or
        // the forward's words of queries qb0 + l32 transposed to this lane's
        // key, query qb0 + 8 g + 4 hi + e at bit 8 g + e after the shift (mode 2)
        uint64_t col_ctr = 0;
        if (DROPOUT == 1)
            col_ctr = p.offset + (uint64_t)(b * p.H + tile_head(it)) * (uint64_t)p.Sq * (uint64_t)p.Sk + (uint64_t)kj;
        const uint32_t km = DROPOUT == 2 ? transpose32(kword, lane) >> (4 * hi) : 0u;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 l4 = *reinterpret_cast<const f32x4*>(lse2 + 8 * g + 4 * hi);
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(dels + 8 * g + 4 * hi);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * g + e;
                const int q = qb0 + 8 * g + 4 * hi + e;
                float pv;
                if constexpr (BIAS)
                    pv = fast_exp2(__builtin_fmaf(sc[r], c, __builtin_fmaf(bias_f32<BT>(bias_at(r)), kLog2e, -l4[e])));
                else
                    pv = fast_exp2(__builtin_fmaf(sc[r], c, -l4[e]));
                if (MASK && q < kj) pv = 0.f;
                // dropout: dropped entries of P and dP become 0; the 1 / (1 - p)
                // of the kept ones goes into dS here and into dV's final scale
                // (a 0 / 1 factor for the regenerated mask and a select for the
                // stored one: the forms that spill least in each instantiation)
                float dpv = dpc[r];
                float pdv = pv;
                if (DROPOUT == 1) {
                    const float z =
                        philox_keep(p.seed, col_ctr + (uint64_t)q * (uint64_t)p.Sk, p.keep_thresh) ? 1.f : 0.f;
                    dpv *= z;
                    pdv *= z;
                } else if (DROPOUT == 2) {
                    const bool keep = ((km >> (8 * g + e)) & 1u) != 0u;
                    dpv = keep ? dpv : 0.f;
                    pdv = keep ? pv : 0.f;
                }
                pd[r] = pdv;
                if constexpr (DFOLD)
                    ds[r] = pv * dpv;  // -dS
                else
                    ds[r] = DROPOUT ? pv * __builtin_fmaf(dpv, p.rp, -d4[e]) : pv * (dpv - d4[e]);
            }
        }
        if (want_db) {
            with_grad_dtype(p.dbias_dtype, [&](auto dt) FA_INLINE {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    store_grad<decltype(dt)::value>(dbrs, ds[r], dbvoff,
                                                    (qb0 + 8 * (r >> 2) + (r & 3)) * (int)p.dbias_ss * p.dbias_es);
            });
        }
        if constexpr (!C::F32) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                bp8[ks] = pack8<T>(pd + 8 * ks);
                bs8[ks] = pack8<T>(ds + 8 * ks);
            }
        }
    };

    // ---- dV^T += dO^T P,  dK^T += Q^T dS for the tile in buffer s ----
    // half H (0 or 1) of the products: query rows [16 H, 16 H + 16)
    auto dkdv_acc = [&](int s, int st, auto half_tag) FA_INLINE {
        constexpr int H2 = decltype(half_tag)::value;
        const T* Qs = (const T*)buf(s) + 32 * st * RW;
        const T* Ds = (const T*)(buf(s) + C::QALLOC) + 32 * st * RW;
        if constexpr (C::F32) {
#pragma unroll
            for (int t = 8 * H2; t < 8 * H2 + 8; ++t) {
                const int qr = 8 * (t >> 2) + 4 * hi + (t & 3);
#pragma unroll
                for (int i = 0; i < DA / 32; ++i) {
                    dv[i] = mfma_f32(Ds[qr * RW + DOFF + 32 * i + l32], pd[t], dv[i]);
                    dk[i] = mfma_f32(Qs[qr * RW + DOFF + 32 * i + l32], ds[t], dk[i]);
                }
            }
        } else {
            // dO^T / Q^T operands straight from the row-major tiles
            const int trow = 4 * hi + ((lane & 15) >> 2);
            const int tcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
            constexpr int ks = H2;
#pragma unroll
                for (int i = 0; i < DA / 32; ++i) {
                    const int off = (16 * ks + trow) * RW + DOFF + 32 * i + tcol;
                    const s16x8 ad = cat4(lds_read_tr16(Ds + off), lds_read_tr16(Ds + off + 8 * RW));
                    const s16x8 aq = cat4(lds_read_tr16(Qs + off), lds_read_tr16(Qs + off + 8 * RW));
                    dv[i] = Elem<T>::mfma(ad, bp8[ks], dv[i]);
                    dk[i] = Elem<T>::mfma(aq, bs8[ks], dk[i]);
                }
        }
    };

    // Loop over query tiles of 64 (two 32-query sub-steps per barrier).  Two
    // LDS buffers alternate: iteration `it` reads tile it (buffer it&1) and
    // copies tile it+1 into the other buffer, last read in iteration it-1,
    // which every wave finished before the opening barrier.  Past the last
    // tile the copy repeats it, which keeps the loop body free of branches.
    // Two workgroups share a CU (255 registers per lane), so each SIMD
    // interleaves the MFMA, softmax and LDS phases of two waves.
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // the forward's keep word of query qb0 + l32 for the wave's 32 keys
    auto load_kbits = [&](int it, int st) FA_INLINE -> uint32_t {
        const int q = tile_q0(it) + 32 * st + l32;
        if (DROPOUT != 2 || q >= p.Sq || kw0 >= p.Sk) return 0u;
        return p.kb[((int64_t)(b * p.H + tile_head(it)) * p.Sq + q) * p.kb_w + (kw0 >> 5)];
    };
    uint32_t kbnext = 0;
    if (total > 0) {
        issue(0, 0);
        load_bias(bnext, 0, 0);
        kbnext = load_kbits(0, 0);
    }
    f32x16 sc, dpc;
    int bcur = 0;  // it & 1
    auto iter = [&](int it, auto mask_tag) FA_INLINE {
        sync_tiles();
        issue(min(it + 1, total - 1), bcur ^ 1);
#pragma unroll
        for (int st = 0; st < C::NSUB; ++st) {
            if constexpr (BIAS) {  // this sub-step's bias; start loading the next one's
#pragma unroll
                for (int r = 0; r < NBI; ++r) braw[r] = bnext[r];
                if (st + 1 < C::NSUB)
                    load_bias(bnext, it, st + 1);
                else
                    load_bias(bnext, min(it + 1, total - 1), 0);
            }
            uint32_t kbits = 0;
            if (DROPOUT == 2) {  // likewise the keep bits
                kbits = kbnext;
                kbnext = st + 1 < C::NSUB ? load_kbits(it, st + 1) : load_kbits(min(it + 1, total - 1), 0);
            }
            sdp(bcur, st, sc, dpc);
            softmax_ds(it, bcur, st, sc, dpc, kbits, mask_tag);
            dkdv_acc(bcur, st, I0{});
            dkdv_acc(bcur, st, I1{});
        }
        bcur ^= 1;
    };
    // dBias rows of query tiles the causal loop skips (queries before the first
    // visited tile) are zero; the visited tiles write every other row
    if (BIAS && CAUSAL && p.dbias != nullptr && p.dbias_zero_fill == 1) {
        const int zrows = min(qt_begin * BQ, p.Sq);
        for (int g = 0; g < p.group; ++g) {
            const __amdgpu_buffer_rsrc_t rs = dbias_buf(hk * p.group + g);
            const int voff = kj < p.Sk ? (hi * (int)p.dbias_ss + kj) * p.dbias_es : kOffNowhere;
            with_grad_dtype(p.dbias_dtype, [&](auto dt) FA_INLINE {
                for (int q = 0; q < zrows; q += 2)
                    store_grad<decltype(dt)::value>(rs, 0.f, voff, q * (int)p.dbias_ss * p.dbias_es);
            });
        }
    }

    // plain tiles first for each query head of the group, then the masked ones
    int it = 0;
    for (int g = 0; g < p.group; ++g) {
        for (; it < g * nq + (nq - n_mask); ++it) iter(it, std::false_type{});
        if (CAUSAL)
            for (; it < (g + 1) * nq; ++it) iter(it, std::true_type{});
    }

    // ---- epilogue: stage dK^T, dV^T through LDS as rows, coalesced stores ----
    constexpr int OW = C::OW;
    constexpr int EPC = 16 / sizeof(T);
    constexpr int CPR = DA / EPC;
    T* Os = (T*)smem + w * 32 * OW;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        sync_tiles();
        const f32x16* acc = pass == 0 ? dk : dv;
        const float mul = pass == 0 ? (DFOLD ? -p.scale : p.scale) : (DROPOUT ? p.rp : 1.f);
#pragma unroll
        for (int i = 0; i < DA / 32; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * i + 8 * g + 4 * hi;  // column DOFF + d of dK / dV
                if constexpr (C::F32) {
                    f32x4 v4;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v4[e] = acc[i][4 * g + e] * mul;
                    *reinterpret_cast<f32x4*>(Os + l32 * OW + d) = v4;
                } else {
                    s16x4 v4;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v4[e] = Elem<T>::pack1(acc[i][4 * g + e] * mul);
                    *reinterpret_cast<s16x4*>(Os + l32 * OW + d) = v4;
                }
            }
        lds_barrier();
        T* gbase = pass == 0 ? (T*)p.dk + b * p.dk_sb + hk * p.dk_sh : (T*)p.dv + b * p.dv_sb + hk * p.dv_sh;
        const int64_t gss = pass == 0 ? p.dk_ss : p.dv_ss;
#pragma unroll
        for (int i = 0; i < 32 * CPR / 64; ++i) {
            const int cidx = lane + 64 * i;
            const int row = cidx / CPR, col = cidx % CPR;
            const int key = kw0 + row;
            if (key < p.Sk)
                *reinterpret_cast<uint4*>(gbase + (int64_t)key * gss + DOFF + col * EPC) =
                    *reinterpret_cast<const uint4*>(Os + row * OW + col * EPC);
        }
    }
}

// ---------------------------------------------------------------------------
// Ping-pong dK/dV for 16-bit inputs without bias or dropout, D = 128, on grids
// that fill the CUs.  One workgroup = 8 waves = 256 keys of one (batch, KV
// head), one workgroup per CU; wave w owns the 32 keys k0 + 32 w ..., whose K
// and V rows it holds in registers (as dkdv_kernel's waves do).  The 64-query
// tiles of Q, dO, LSE * log2 e and delta are consumed as two 32-query
// sub-steps, one per round; every wave runs, for each round r,
//   M(r): dV += dO^T P(r-1), dK += Q^T dS(r-1), then S(r) = Q K^T, dP(r) = dO V^T
//   V(r): P(r) = exp2(S c - LSE), dS(r) = P (dP - delta), packed to 16 bits
// with a workgroup barrier after each phase, but waves 4-7 pass one extra
// barrier first (and waves 0-3 one at the end).  Waves w and w + 4 share a
// SIMD (the hardware deals the waves of a workgroup to SIMDs 0, 2, 1, 3, 0, 2,
// 1, 3), so the two run one phase apart: one's matrix products overlap the
// other's softmax arithmetic.
// Tile copies (direct to LDS) stall the issuing wave while the CU's vector
// memory path takes them (about 64 bytes a clock), so they are spread thin:
// each tile is shared by 256 keys, and each wave issues 3 copy instructions
// in each of its V phases -- waves 0-3 the Q rows and LSE row of tile
// (r + 3) / 2, waves 4-7 the dO rows and delta row of tile (r + 4) / 2 (one
// half of the tile's 24 instructions per round, the LSE / delta row copied
// twice so every wave issues the same number).  Tiles rotate through three
// LDS slots: tile j replaces tile j - 3, whose last reader, the M phase of
// round 2 j - 4 of waves 4-7, precedes the first copy of tile j (V phase of
// round 2 j - 4 of waves 4-7, round 2 j - 3 of waves 0-3).  At the end of its
// V phase a wave waits until its copies of earlier rounds have landed, which
// covers tile j before the barrier that opens M(2 j) of waves 0-3.  Per
// element the arithmetic is that of dkdv_kernel, in the same order (each
// key's dK / dV accumulate its query tiles in the same sequence), so the
// outputs are bit-identical to it.
template <typename T, int D>
struct DkdvPPCfg {
    static constexpr int NW = 8;
    static constexpr int NT = 64 * NW;
    static constexpr int BK = 32 * NW;               // keys per workgroup
    static constexpr int BQ = 64;                    // queries per tile: two 32-query sub-steps
    static constexpr int RW = D + 24;                // Q / dO row stride, as in dkdv_kernel
    static constexpr int QALLOC = BQ * RW * (int)sizeof(T);
    // per slot: Q rows, dO rows, then LSE * log2 e [BQ] and delta [BQ] as floats
    static constexpr int SLOT_BYTES = 2 * QALLOC + 2 * BQ * 4;
    static constexpr int NSLOT = 3;
    static constexpr int SMEM_BYTES = NSLOT * SLOT_BYTES;
    static constexpr int EPC = 16 / (int)sizeof(T);
    static constexpr int CW = RW / EPC;              // 16-byte chunks per LDS row
    static constexpr int NI = BQ * CW / 64;          // copy instructions per tile and matrix (all 64 lanes)
    static_assert((BQ * CW) % 64 == 0, "whole copy instructions");
    // a group's items per tile: NI row copies + the LSE / delta row, dealt as
    // item 8 n + 4 hf + w4 to wave w4 of the group in the V phase of half hf:
    // 3 items per wave in half 0, 2 in half 1
    static_assert(NI + 1 == 20, "20 items per group and tile");
    static constexpr int OW = D + 8;                 // output staging row stride
    static_assert(SMEM_BYTES <= 160 * 1024, "LDS of one CU");
    static_assert(NW * 32 * OW * (int)sizeof(T) <= SMEM_BYTES, "output staging");
    static_assert(SLOT_BYTES % 16 == 0, "16-byte aligned slots");
};

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(512, 1) void dkdv_pp_kernel(const BwdParams p, const int n_ktiles) {
    using C = DkdvPPCfg<T, D>;
    static_assert(!Elem<T>::kF32 && D == 128, "16-bit inputs, D = 128");
    constexpr int BQ = C::BQ, RW = C::RW;
    __shared__ __attribute__((aligned(16))) char smem[C::SMEM_BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), l32 = lane & 31, hi = lane >> 5;
    const int grp = w >> 2, w4 = w & 3;
    const int2 tord = tile_order<32, CAUSAL>(n_ktiles);
    const int bhk = tord.x;
    const int kt = tord.y;
    const int hk = bhk % p.Hkv, b = bhk / p.Hkv;
    const int k0 = kt * C::BK;
    const int kw0 = k0 + 32 * w;
    const int kj = kw0 + l32;  // this lane's key

    // ---- K, V rows of this lane's key in registers (MFMA B operands) ----
    constexpr int KR = D / 16;
    uint4 kreg[KR], vreg[KR];
    {
        const T* krow = (const T*)p.k + b * p.k_sb + (int64_t)kj * p.k_ss + hk * p.k_sh;
        const T* vrow = (const T*)p.v + b * p.v_sb + (int64_t)kj * p.v_ss + hk * p.v_sh;
        const bool ok = kj < p.Sk;
#pragma unroll
        for (int i = 0; i < KR; ++i) {
            const int d0 = 16 * i + 8 * hi;
            kreg[i] = ok ? *reinterpret_cast<const uint4*>(krow + d0) : make_uint4(0u, 0u, 0u, 0u);
            vreg[i] = ok ? *reinterpret_cast<const uint4*>(vrow + d0) : make_uint4(0u, 0u, 0u, 0u);
        }
        // -V: the dP products start from delta and give delta - dP (as dkdv_kernel)
#pragma unroll
        for (int i = 0; i < KR; ++i) vreg[i] = neg16x8(vreg[i]);
    }
    f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) { dk[i] = f32x16{}; dv[i] = f32x16{}; }
    const float c = p.scale_log2;

    // the run of tiles: per query head of the KV group, the query tiles from
    // the last one down to the first that reaches the workgroup's keys (as in
    // dkdv_kernel: the workgroups of a head read the same tiles together)
    const int qt_begin = CAUSAL ? (k0 / BQ) : 0;
    const int qt_end = (p.Sq + BQ - 1) / BQ;
    const int nq = qt_end > qt_begin ? qt_end - qt_begin : 0;
    const int total = nq * p.group;  // tiles; rounds = 2 * total
    // position of a round's tile in the run (tile in the head's run, LDS
    // slot), advanced one tile at a time: no integer division in the loop
    struct Pos {
        int i, s;
    };
    auto advance = [&](Pos& t) FA_INLINE {
        if (++t.i == nq) t.i = 0;
        if (++t.s == C::NSLOT) t.s = 0;
    };
    auto pos_q0 = [&](const Pos& t) FA_INLINE { return (qt_end - 1 - t.i) * BQ; };
    auto slot = [&](int s) FA_INLINE -> char* { return smem + s * C::SLOT_BYTES; };
    // this wave's sub-step (first query qs0): any visible (query, key) pair,
    // and any masked one
    auto active = [&](int qs0) FA_INLINE { return !CAUSAL || qs0 + 31 >= kw0; };
    auto masked = [&](int qs0) FA_INLINE { return CAUSAL && qs0 < kw0 + 31; };

    // ---- tile copies: waves 0-3 Q rows (+ LSE), waves 4-7 dO rows (+ delta) ----
    // The wave's source base, strides and the workspace base are formed once
    // and kept opaque (scalar registers): otherwise the compiler re-reads the
    // kernel arguments inside the loop (a scalar memory load and a wait for
    // it, and for every LDS access in flight, per round).
    auto opaque64 = [](uint64_t x) FA_INLINE {
        asm volatile("" : "+s"(x));
        return x;
    };
    auto opaque32 = [](uint32_t x) FA_INLINE {
        asm volatile("" : "+s"(x));
        return x;
    };
    const int64_t css = grp == 0 ? p.q_ss : p.do_ss;  // row stride (elements)
    const uint64_t cbase = opaque64((uint64_t)(uintptr_t)(grp == 0 ? (const T*)p.q + b * p.q_sb
                                                                   : (const T*)p.dout + b * p.do_sb));
    const uint64_t crow = opaque64((uint64_t)css * sizeof(T));                             // bytes per row
    const uint64_t chead = opaque64((uint64_t)(grp == 0 ? p.q_sh : p.do_sh) * sizeof(T));  // bytes per head
    const uint64_t wbase = opaque64((uint64_t)(uintptr_t)(p.lse2 + (int64_t)b * p.H * p.ws_stride));
    const uint32_t wrow_bytes = opaque32((uint32_t)p.ws_stride * 4u);
    const uint32_t full_bytes = opaque32((uint32_t)(((BQ - 1) * (int)css + D) * (int)sizeof(T)));
    const uint32_t woff = 4u * (uint32_t)(grp * p.sq_pad + lane);
    const int q_rows = p.Sq;
    // per-lane source offsets of the wave's row-copy items 8 n + 4 hf + w4
    // (instruction g covers LDS chunks 64 g ..; padding chunks read nothing)
    int coff[2][3];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int n = 0; n < 3; ++n) {
            const int cidx = 64 * (8 * n + 4 * hf + w4) + lane;
            const int row = cidx / C::CW, col = cidx % C::CW;
            coff[hf][n] = col < D / C::EPC ? (row * (int)css + col * C::EPC) * (int)sizeof(T) : kOffNowhere;
        }
    // The copy position: the current tile's sources and ranges (rows and the
    // workspace row) and LDS slot, advanced one tile at a time by additions:
    // within a head's run the tiles step down by BQ rows and only the first
    // tile of a run (the last rows) can be partial.
    struct Cp {
        uint64_t src, hsrc, wsrc, hwsrc;
        uint32_t bytes, wbytes, lds;
        int i;
    };
    const int qb0_first = (qt_end - 1) * BQ;
    const uint32_t bytes_first = opaque32(
        q_rows - qb0_first >= BQ ? full_bytes : (uint32_t)(((q_rows - qb0_first - 1) * (int)css + D) * (int)sizeof(T)));
    const uint32_t wbytes_first = opaque32(wrow_bytes - 4u * (uint32_t)qb0_first);
    const uint64_t dsrc = opaque64((uint64_t)BQ * crow);
    const uint32_t lds_first = __builtin_amdgcn_readfirstlane(lds_addr(smem + grp * C::QALLOC));
    const uint32_t lds_wrap = lds_first + C::NSLOT * C::SLOT_BYTES;
    const uint32_t lse_off = (uint32_t)((2 - grp) * C::QALLOC + grp * 4 * BQ);  // the workspace row's LDS offset
    Cp c0;
    c0.hsrc = opaque64(cbase + (uint64_t)(int64_t)qb0_first * crow + (uint64_t)(hk * p.group) * chead);
    c0.src = c0.hsrc;
    c0.hwsrc = opaque64(wbase + (uint64_t)(hk * p.group) * wrow_bytes + 4u * (uint32_t)qb0_first);
    c0.wsrc = c0.hwsrc;
    c0.bytes = bytes_first;
    c0.wbytes = wbytes_first;
    c0.lds = lds_first;
    c0.i = 0;
    auto advance_cp = [&](Cp& t) FA_INLINE {
        if (++t.i == nq) {
            t.i = 0;
            t.hsrc += chead;
            t.hwsrc += wrow_bytes;
            t.src = t.hsrc;
            t.wsrc = t.hwsrc;
            t.bytes = bytes_first;
            t.wbytes = wbytes_first;
        } else {
            t.src -= dsrc;
            t.wsrc -= 4u * BQ;
            t.bytes = full_bytes;
            t.wbytes += 4u * BQ;
        }
        t.lds += C::SLOT_BYTES;
        if (t.lds == lds_wrap) t.lds = lds_first;
    };
    // half hf of the tile at t: the wave's items 8 n + 4 hf + w4 of the group's 20
    auto issue = [&](const Cp& t, int hf) FA_INLINE {
        u32x4 rs;
        rs[0] = (uint32_t)t.src;
        rs[1] = (uint32_t)(t.src >> 32) & 0xFFFFu;
        rs[2] = t.bytes;
        rs[3] = 0x00020000u;
        const uint32_t l0 = t.lds;
        auto items = [&](auto hf_tag) FA_INLINE {
            constexpr int HF = decltype(hf_tag)::value;
#pragma unroll
            for (int n = 0; n < 3; ++n) {
                const int g = 8 * n + 4 * HF + w4;  // wave-uniform
                if (g < C::NI) {
                    dma_load16_untracked(rs, __builtin_amdgcn_readfirstlane(l0 + 1024 * g), coff[HF][n]);
                } else if (g == C::NI) {  // the LSE (waves 0-3) or delta (waves 4-7) row, one dword per lane
                    u32x4 ws;  // (rows qb0 .. qb0 + BQ <= sq_pad)
                    ws[0] = (uint32_t)t.wsrc;
                    ws[1] = (uint32_t)(t.wsrc >> 32) & 0xFFFFu;
                    ws[2] = t.wbytes;
                    ws[3] = 0x00020000u;
                    dma_load4_untracked(ws, __builtin_amdgcn_readfirstlane(l0 + lse_off), woff);
                }
            }
        };
        if (hf == 0)
            items(std::integral_constant<int, 0>{});
        else
            items(std::integral_constant<int, 1>{});
    };

    // ---- M phase: dV/dK of the previous sub-step, then S/dP of this one ----
    // dV/dK step t (t = ks (D / 32) + i): dO^T, Q^T of query rows 16 ks .. of
    // the sub-step, d block i (transposing reads); S/dP step kk: the Q, dO row
    // fragments d = 16 kk + 8 hi of query row l32.  The LDS operands of step
    // t + MP are read during step t.
    const int trow = 4 * hi + ((lane & 15) >> 2);
    const int tcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    constexpr int NA = 2 * (D / 32);  // dV/dK steps (a dV and a dK product each)
    constexpr int NSTEP = NA + D / 16;
    constexpr int MP = 2;
    s16x8 bp8[2], bs8[2];  // P, dS of the previous sub-step (B operands)
    f32x16 sc, dpc;
    // A: dV/dK of the sub-step in slot sa / rows sta; BB: S/dP of the one in slot sb / rows stb
    auto mphase = [&](int sa, int sta, int sb, int stb, auto a_tag, auto b_tag) FA_INLINE {
        constexpr bool A = decltype(a_tag)::value, BB = decltype(b_tag)::value;
        const T* Qa = (const T*)slot(sa) + 32 * sta * RW;
        const T* Da = (const T*)(slot(sa) + C::QALLOC) + 32 * sta * RW;
        const T* Qb = (const T*)slot(sb) + (32 * stb + l32) * RW + 8 * hi;
        const T* Db = (const T*)(slot(sb) + C::QALLOC) + (32 * stb + l32) * RW + 8 * hi;
        const float* delb = (const float*)(slot(sb) + 2 * C::QALLOC) + BQ + 32 * stb;
        s16x8 x[NSTEP], y[NSTEP];
        f32x16 dinit;  // delta of the sub-step's queries: the dP products start from it
        auto rd = [&](int t) FA_INLINE {
            if (t < NA) {
                const int ks = t / (D / 32), i = t % (D / 32);
                const int off = (16 * ks + trow) * RW + 32 * i + tcol;
                x[t] = cat4(lds_read_tr16(Da + off), lds_read_tr16(Da + off + 8 * RW));
                y[t] = cat4(lds_read_tr16(Qa + off), lds_read_tr16(Qa + off + 8 * RW));
            } else {
                const int kk = t - NA;
                x[t] = *reinterpret_cast<const s16x8*>(Qb + 16 * kk);
                y[t] = *reinterpret_cast<const s16x8*>(Db + 16 * kk);
                if (kk == 0) dinit = delta16(delb, hi);
            }
        };
        auto mm = [&](int t) FA_INLINE {
            if (t < NA) {
                const int ks = t / (D / 32), i = t % (D / 32);
                dv[i] = Elem<T>::mfma(x[t], bp8[ks], dv[i]);
                dk[i] = Elem<T>::mfma(y[t], bs8[ks], dk[i]);
            } else {
                const int kk = t - NA;
                sc = Elem<T>::mfma(x[t], __builtin_bit_cast(s16x8, kreg[kk]), kk == 0 ? f32x16{} : sc);
                dpc = Elem<T>::mfma(y[t], __builtin_bit_cast(s16x8, vreg[kk]), kk == 0 ? dinit : dpc);
            }
        };
        constexpr int T0 = A ? 0 : NA, T1 = BB ? NSTEP : NA;
#pragma unroll
        for (int t = T0; t < T0 + MP; ++t) rd(t);
#pragma unroll
        for (int t = T0; t < T1; ++t) {
            if (t + MP < T1) rd(t + MP);
            mm(t);
        }
        // the same order for the scheduler: reads of MP steps, then per step
        // its two products followed by the reads of step t + MP
        auto rd_group = [&](int t) FA_INLINE {  // 4 transposing reads or 2 row reads
            if (t < NA)
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
            else if (t == NA)
                __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);  // with the 4 delta reads
            else
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        };
#pragma unroll
        for (int t = T0; t < T0 + MP; ++t) rd_group(t);
#pragma unroll
        for (int t = T0; t < T1; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            if (t + MP < T1) rd_group(t + MP);
        }
    };

    // ---- V phase: P, dS of the sub-step (rows st of the tile in slot s) ----
    // On a sub-step that straddles the diagonal (msk), the entries of queries
    // below this lane's key are then zeroed in place (one code path: branches
    // that each produce P / dS make the register allocator spill)
    auto vphase = [&](int s, int st, int qs0, bool msk) FA_INLINE {
        const float* lse2 = (const float*)(slot(s) + 2 * C::QALLOC) + 32 * st;
        float pd[16], ds[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 l4 = *reinterpret_cast<const f32x4*>(lse2 + 8 * g + 4 * hi);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int rr = 4 * g + e;
                const float pv = fast_exp2(__builtin_fmaf(sc[rr], c, -l4[e]));
                pd[rr] = pv;
                ds[rr] = pv * dpc[rr];  // -dS (dpc = delta - dP)
            }
        }
        if (CAUSAL && msk) {
            // query qs0 + 8 g + 4 hi + e is masked when 8 g + e < dlt (one
            // per-lane value against constants)
            const int dlt = kj - 4 * hi - qs0;
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (8 * g + e < dlt) {
                        pd[4 * g + e] = 0.f;
                        ds[4 * g + e] = 0.f;
                    }
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            bp8[ks] = pack8<T>(pd + 8 * ks);
            bs8[ks] = pack8<T>(ds + 8 * ks);
        }
    };

    auto sched_fence = [&]() FA_INLINE { __builtin_amdgcn_sched_barrier(0); };
    using TT = std::true_type;
    using FF = std::false_type;

    // prologue: tiles 0 and 1, every wave its group's 6 instructions of each
    {
        Cp t = c0;
        for (int j = 0; j < 2; ++j) {
            if (j < total) {
                issue(t, 0);
                issue(t, 1);
            }
            advance_cp(t);
        }
    }
    wait_vmem();
    lds_barrier();
    if (grp == 1) barrier_no_fence();  // waves 4-7 run one phase behind

    // V phase of round r (tile pr, sub-step st): this round's copies -- half
    // (m & 1) of tile m / 2, m = r + 3 (waves 0-3) or r + 4 (waves 4-7), tiles
    // 2 .. total - 1 (the prologue copied 0 and 1) -- then P, dS (zero where
    // the sub-step has no visible pair or there is no sub-step), then wait for
    // this wave's copies of earlier rounds.  The slot schedule is modelled for
    // every run length up to 100 tiles by tests/test_pp_schedule_cpu.py.
    Cp pc = c0;  // tile m / 2 of the copies
    advance_cp(pc);
    if (grp == 1) advance_cp(pc);  // round 0: tile 1 (waves 0-3, nothing to copy) or 2 (waves 4-7)
    auto vround = [&](int r, const Pos& pr, int st, bool act) FA_INLINE {
        const int m = r + 3 + grp;
        const int j = m >> 1;
        const bool cp = j >= 2 && j < total;
        if (cp) issue(pc, m & 1);
        if (m & 1) advance_cp(pc);
        if (act) {
            const int qs0 = pos_q0(pr) + 32 * st;
            vphase(pr.s, st, qs0, masked(qs0));
        } else {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                bp8[ks] = s16x8{};
                bs8[ks] = s16x8{};
            }
        }
        if (!cp)
            wait_vmem();
        else if ((m & 1) == 0)
            wait_vmem_below<3>();
        else
            wait_vmem_below<2>();
    };
    // Round 0 runs S/dP only; rounds 1 .. 2 total run both halves of the M
    // phase unconditionally (one code path keeps the accumulators in place): a
    // sub-step without visible pairs gets P = dS = 0, and the S/dP products of
    // round 2 total (no sub-step) are not used.  Idle products cost no time,
    // as the workgroup's waves run in lock step.
    if (total > 0) {
        Pos pr{0, 0};  // tile of round r
        sched_fence();
        mphase(0, 0, 0, 0, FF{}, TT{});
        sched_fence();
        barrier_no_fence();
        sched_fence();
        vround(0, pr, 0, active(pos_q0(pr)));
        sched_fence();
        barrier_no_fence();
        int s_prev = 0;
        for (int r = 1; r <= 2 * total; ++r) {
            const int st = r & 1;
            if (st == 0) advance(pr);
            sched_fence();
            mphase(s_prev, st ^ 1, pr.s, st, TT{}, TT{});
            sched_fence();
            barrier_no_fence();
            sched_fence();
            vround(r, pr, st, r < 2 * total && active(pos_q0(pr) + 32 * st));
            sched_fence();
            barrier_no_fence();
            s_prev = pr.s;
        }
    }
    if (grp == 0) barrier_no_fence();
    sched_fence();

    // ---- epilogue: stage dK^T, dV^T through LDS as rows, coalesced stores ----
    // (every M phase is done: the last barrier follows M(2 total) of waves 4-7)
    constexpr int OW = C::OW;
    constexpr int EPC = 16 / sizeof(T);
    constexpr int CPR = D / EPC;
    T* Os = reinterpret_cast<T*>(smem) + w * 32 * OW;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1) lds_barrier();  // this wave's dK rows are stored (its own region)
        const f32x16* acc = pass == 0 ? dk : dv;
        const float mul = pass == 0 ? -p.scale : 1.f;  // the products summed -dS
#pragma unroll
        for (int i = 0; i < D / 32; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                s16x4 v4;
#pragma unroll
                for (int e = 0; e < 4; ++e) v4[e] = Elem<T>::pack1(acc[i][4 * g + e] * mul);
                *reinterpret_cast<s16x4*>(Os + l32 * OW + 32 * i + 8 * g + 4 * hi) = v4;
            }
        lds_barrier();
        T* gbase = pass == 0 ? (T*)p.dk + b * p.dk_sb + hk * p.dk_sh : (T*)p.dv + b * p.dv_sb + hk * p.dv_sh;
        const int64_t gss = pass == 0 ? p.dk_ss : p.dv_ss;
#pragma unroll
        for (int i = 0; i < 32 * CPR / 64; ++i) {
            const int cidx = lane + 64 * i;
            const int row = cidx / CPR, col = cidx % CPR;
            const int key = kw0 + row;
            if (key < p.Sk)
                *reinterpret_cast<uint4*>(gbase + (int64_t)key * gss + col * EPC) =
                    *reinterpret_cast<const uint4*>(Os + row * OW + col * EPC);
        }
    }
}

// ---------------------------------------------------------------------------
// dK/dV with K and V in LDS (16-bit inputs, D >= 64, no dropout): for grids
// of fewer workgroups than CUs, and with a bias at every grid size (the
// bias's registers do not fit two workgroups of dkdv_kernel per CU at D = 128).
// One workgroup = 8 waves = 128 keys of one (batch, KV head), one workgroup per
// CU.  Waves w and w + 4 share a SIMD and the 32 keys k0 + 32 (w % 4) ..: each
// takes one of the two 32-query sub-steps of every 64-query tile, and their
// dK / dV partials are summed through LDS at the end.  With the keys' K and V
// rows read from LDS (B operands, row reads) instead of held in registers, a
// wave keeps 64 registers for operand prefetch: the S / dP products and the
// dV / dK products each run with their LDS reads two steps ahead, as two
// independent accumulator chains, instead of one MFMA per LDS latency.  Tiles
// of Q, dO, LSE and delta stream as in dkdv_kernel.
// With a bias (TB) each wave loads its sub-step's bias values of the next
// tile once its softmax is done (one set of registers), and the tile barrier
// waits only for the copies: those loads stay in flight across it.  dBias
// (= dS) is stored as in dkdv_kernel; the zeros of the causal gradient are
// written by the dQ pass (dbias_zero_fill == 2) or by the reduction.
template <typename T, int D>
struct Dkdv8Cfg {
    static constexpr int NW = 8;
    static constexpr int NT = 64 * NW;
    static constexpr int BK = 128;                  // keys per workgroup
    static constexpr int BQ = 64;                   // queries per tile
    static constexpr int RW = D + (D == 64 ? 8 : 24);  // Q / dO rows, as in DkdvCfg
    static constexpr int KVW = D + 8;               // K / V rows (conflict-free b128 row reads)
    static constexpr int QALLOC = BQ * RW * (int)sizeof(T);
    static constexpr int BUF_BYTES = 2 * QALLOC + 2 * BQ * 4;
    static constexpr int NBUF = 2;
    static constexpr int KV_BYTES = BK * KVW * (int)sizeof(T);
    static constexpr int SMEM_BYTES = 2 * KV_BYTES + NBUF * BUF_BYTES;
    static constexpr int OW = D + 8;                // output staging stride
    // waves 4-7 hand their dK, dV (fp32) to waves 0-3 through LDS
    static constexpr int MERGE_BYTES = 4 * 64 * 2 * (D / 32) * 16 * 4;
    static_assert(MERGE_BYTES <= SMEM_BYTES && 4 * 32 * OW * (int)sizeof(T) <= SMEM_BYTES, "epilogue fits");
    static_assert(SMEM_BYTES <= 160 * 1024, "LDS of one CU");
    using Rows = DmaRowGroups<T, BQ, D, RW, 4>;     // waves 0-3: Q rows, waves 4-7: dO rows
    using KV = DmaTile<T, BK, D, KVW, NW>;
};

// (bid, nblocks: this workgroup among the dK/dV ones; smem: Dkdv8Cfg::SMEM_BYTES of LDS)
template <typename T, int D, bool CAUSAL, typename TB>
__device__ FA_INLINE inline void dkdv8_body(const BwdParams& p, const int n_ktiles, const int bid, const int nblocks,
                                           char* smem) {
    using C = Dkdv8Cfg<T, D>;
    static_assert(!Elem<T>::kF32, "16-bit inputs");
    constexpr bool BIAS = !std::is_void<TB>::value;
    using BT = typename std::conditional<BIAS, TB, T>::type;
    constexpr int BQ = C::BQ, RW = C::RW, KVW = C::KVW;

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), l32 = lane & 31, hi = lane >> 5;
    const int kb = w & 3;   // key block
    const int st = w >> 2;  // query sub-step of every tile
    const int2 tord = tile_order<32, CAUSAL>(n_ktiles, bid, nblocks);  // kt = 0 sees the most queries
    const int kt = tord.y;
    const int2 sbh = slice_bh(tord.x, p.Hkv, p.B, BIAS && p.bias_sb == 0);
    const int hk = sbh.y, b = sbh.x;
    const int k0 = kt * C::BK;
    const int kw0 = k0 + 32 * kb;
    const int kj = kw0 + l32;  // this lane's key

    T* Ks = reinterpret_cast<T*>(smem);
    T* Vs = reinterpret_cast<T*>(smem + C::KV_BYTES);
    char* bufs = smem + 2 * C::KV_BYTES;
    {  // K and V rows of the 128 keys (rows past Sk land as zeros)
        typename C::KV kd;
        kd.init(p.k_ss, lane, w);
        kd.load_untracked((const T*)p.k + b * p.k_sb + (int64_t)k0 * p.k_ss + hk * p.k_sh, p.k_ss, p.Sk - k0, Ks, lane);
        typename C::KV vd;
        vd.init(p.v_ss, lane, w);
        vd.load_untracked((const T*)p.v + b * p.v_sb + (int64_t)k0 * p.v_ss + hk * p.v_sh, p.v_ss, p.Sk - k0, Vs, lane);
    }

    f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) { dk[i] = f32x16{}; dv[i] = f32x16{}; }
    const float c = p.scale_log2;

    // query tiles as in dkdv_kernel: per query head of the group from the last
    // one down; the final tiles of each run cross this wave's keys (masked)
    const int qt_begin = CAUSAL ? (k0 / BQ) : 0;
    const int qt_end = (p.Sq + BQ - 1) / BQ;
    const int nq = qt_end > qt_begin ? qt_end - qt_begin : 0;
    const int total = nq * p.group;
    const int n_mask = CAUSAL ? min(nq, max(0, (kw0 + 31 + BQ - 1) / BQ - qt_begin)) : 0;

    const bool copy_q = w < 4;
    typename C::Rows rows;
    rows.init(copy_q ? p.q_ss : p.do_ss, lane, w & 3);
    auto buf = [&](int s) -> char* { return bufs + s * C::BUF_BYTES; };
    auto tile_head = [&](int it) { return hk * p.group + it / nq; };
    auto tile_q0 = [&](int it) { return (qt_end - 1 - it % nq) * BQ; };
    auto issue = [&](int it, int s) FA_INLINE {
        const int hh = tile_head(it), qb0 = tile_q0(it);
        char* bp = buf(s);
        const T* src = copy_q ? (const T*)p.q + b * p.q_sb + (int64_t)qb0 * p.q_ss + hh * p.q_sh
                              : (const T*)p.dout + b * p.do_sb + (int64_t)qb0 * p.do_ss + hh * p.do_sh;
        rows.load_untracked(src, copy_q ? p.q_ss : p.do_ss, p.Sq - qb0, (const T*)(bp + (copy_q ? 0 : C::QALLOC)));
        // every wave copies the LSE / delta rows (the same values)
        const float* wrow = p.lse2 + ((int64_t)b * p.H + hh) * p.ws_stride + qb0;
        const u32x4 rs = buffer_words(wrow, (p.ws_stride - qb0) * 4);
        const uint32_t f = lds_addr(bp + 2 * C::QALLOC);
        dma_load4_untracked(rs, f, 4 * lane);
        dma_load4_untracked(rs, f + 4 * BQ, 4 * (p.sq_pad + lane));
    };
    auto sync_tiles = [&]() {
        wait_vmem();
        lds_barrier();
    };
    // the loop's barrier: the copies of the tile are done once at most the
    // NBL bias loads issued after them are in flight (vector loads complete in
    // order; the dBias stores, issued before the copies, only add to the
    // count).  A partial wait may count only loads issued after the ones it
    // guards: issued after the copies and counted in the wait, the dS stores
    // gave NaN in dK and dBias at B=4, S=4096 (the barrier passed with copies
    // in flight; stores evidently complete out of order with respect to loads)
    constexpr int NBL = BIAS ? 16 : 0;
    auto sync_copies = [&]() {
        wait_vmem_below<NBL>();
        barrier_no_fence();
    };

    // ---- bias of this lane's key for the 16 queries {8 g + 4 hi + e} of the sub-step ----
    // (as in dkdv_kernel: rows past Sq read zeros, lanes past Sk read zeros or
    // another row and are never stored; 16-bit values two to a register)
    constexpr bool B16 = BIAS && !Elem<BT>::kF32;
    constexpr int NBI = BIAS ? (B16 ? 8 : 16) : 1;
    using BR = typename std::conditional<B16, s16x2, float>::type;
    BR braw[NBI];
    const int bvoff = (4 * hi * (int)p.bias_ss + kj) * (int)sizeof(BT);
    auto load_bias = [&](int it) FA_INLINE {
        if constexpr (BIAS) {
            const __amdgpu_buffer_rsrc_t rs =
                slice_buffer((const BT*)p.bias + b * p.bias_sb + tile_head(it) * p.bias_sh, p.bias_span);
            const int qb0 = tile_q0(it) + 32 * st;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const auto x = load_bias1<BT>(rs, bvoff, (qb0 + 8 * (r >> 2) + (r & 3)) * (int)p.bias_ss * (int)sizeof(BT));
                if constexpr (B16)
                    braw[r >> 1][r & 1] = x;
                else
                    braw[r] = x;
            }
        }
    };
    auto bias_at = [&](int r) FA_INLINE {
        if constexpr (B16)
            return braw[r >> 1][r & 1];
        else
            return braw[r];
    };
    const int dbvoff = kj < p.Sk ? (4 * hi * (int)p.dbias_ss + kj) * p.dbias_es : kOffNowhere;

    // ---- S = Q K^T, dP = dO V^T for this wave's sub-step (C[q][key]) ----
    // step t: the t-th 16-wide slice of D; reads of step t + 2 during step t
    constexpr int NK = D / 16;
    f32x16 sc, dpc;
    auto sdp = [&](int s) FA_INLINE {
        const T* Qs = (const T*)buf(s) + (32 * st + l32) * RW + 8 * hi;
        const T* Ds = (const T*)(buf(s) + C::QALLOC) + (32 * st + l32) * RW + 8 * hi;
        const T* kr = Ks + (32 * kb + l32) * KVW + 8 * hi;
        const T* vr = Vs + (32 * kb + l32) * KVW + 8 * hi;
        s16x8 aq[NK], ak[NK], ad[NK], av[NK];
        auto rd = [&](int t) FA_INLINE {
            aq[t] = *reinterpret_cast<const s16x8*>(Qs + 16 * t);
            ak[t] = *reinterpret_cast<const s16x8*>(kr + 16 * t);
            ad[t] = *reinterpret_cast<const s16x8*>(Ds + 16 * t);
            av[t] = *reinterpret_cast<const s16x8*>(vr + 16 * t);
        };
        rd(0);
        rd(1);
#pragma unroll
        for (int t = 0; t < NK; ++t) {
            if (t + 2 < NK) rd(t + 2);
            sc = Elem<T>::mfma(aq[t], ak[t], t == 0 ? f32x16{} : sc);
            dpc = Elem<T>::mfma(ad[t], av[t], t == 0 ? f32x16{} : dpc);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
        for (int t = 0; t < NK; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            if (t + 2 < NK) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        }
    };

    // ---- P and dS (scale applied at the end) ----
    s16x8 bp8[2], bs8[2];
    auto softmax_ds = [&](int it, int s, auto mask_tag) FA_INLINE {
        constexpr bool MASK = decltype(mask_tag)::value;
        const float* lse2 = (const float*)(buf(s) + 2 * C::QALLOC) + 32 * st;
        const float* dels = lse2 + BQ;
        const int qb0 = tile_q0(it) + 32 * st;
        float pd[16], ds[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 l4 = *reinterpret_cast<const f32x4*>(lse2 + 8 * g + 4 * hi);
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(dels + 8 * g + 4 * hi);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * g + e;
                float pv;
                if constexpr (BIAS)
                    pv = fast_exp2(__builtin_fmaf(sc[r], c, __builtin_fmaf(bias_f32<BT>(bias_at(r)), kLog2e, -l4[e])));
                else
                    pv = fast_exp2(__builtin_fmaf(sc[r], c, -l4[e]));
                if (MASK && qb0 + 8 * g + 4 * hi + e < kj) pv = 0.f;
                pd[r] = pv;
                ds[r] = pv * (dpc[r] - d4[e]);
            }
        }
        if (BIAS && p.dbias != nullptr) {
            const __amdgpu_buffer_rsrc_t dbrs = slice_buffer(
                (const char*)p.dbias + (b * p.dbias_sb + tile_head(it) * p.dbias_sh) * p.dbias_es, p.dbias_span);
            with_grad_dtype(p.dbias_dtype, [&](auto dt) FA_INLINE {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    store_grad<decltype(dt)::value>(dbrs, ds[r], dbvoff,
                                                    (qb0 + 8 * (r >> 2) + (r & 3)) * (int)p.dbias_ss * p.dbias_es);
            });
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            bp8[ks] = pack8<T>(pd + 8 * ks);
            bs8[ks] = pack8<T>(ds + 8 * ks);
        }
    };

    // ---- dV^T += dO^T P, dK^T += Q^T dS (A operands by transposing reads) ----
    auto dkdv_acc = [&](int s) FA_INLINE {
        const int trow = 4 * hi + ((lane & 15) >> 2);
        const int tcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
        const T* Qs = (const T*)buf(s) + (32 * st + trow) * RW + tcol;
        const T* Ds = (const T*)(buf(s) + C::QALLOC) + (32 * st + trow) * RW + tcol;
        constexpr int NS = 2 * (D / 32);  // steps: (ks, i)
        s16x8 ad[NS], aq[NS];
        auto rd = [&](int t) FA_INLINE {
            const int ks = t / (D / 32), i = t % (D / 32);
            const int off = 16 * ks * RW + 32 * i;
            ad[t] = cat4(lds_read_tr16(Ds + off), lds_read_tr16(Ds + off + 8 * RW));
            aq[t] = cat4(lds_read_tr16(Qs + off), lds_read_tr16(Qs + off + 8 * RW));
        };
        rd(0);
        rd(1);
#pragma unroll
        for (int t = 0; t < NS; ++t) {
            const int ks = t / (D / 32), i = t % (D / 32);
            if (t + 2 < NS) rd(t + 2);
            dv[i] = Elem<T>::mfma(ad[t], bp8[ks], dv[i]);
            dk[i] = Elem<T>::mfma(aq[t], bs8[ks], dk[i]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
        for (int t = 0; t < NS; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            if (t + 2 < NS) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        }
    };

    if (total > 0) {
        issue(0, 0);
        load_bias(0);
    }
    int bcur = 0;
    // Without a bias the next tile's copy starts right after the barrier.
    // With one it starts after the softmax, followed by the next bias loads:
    // the compiler makes the first use of a bias value wait until no vector
    // load it knows of issued after that value's load is pending (vmcnt(0)),
    // which would also drain a copy issued before that use.  Past the last
    // tile the copy and the loads repeat it (never used), which keeps the
    // count of loads behind the copy fixed.
    auto iter = [&](int it, auto mask_tag) FA_INLINE {
        sync_copies();
        if constexpr (!BIAS) issue(min(it + 1, total - 1), bcur ^ 1);
        sdp(bcur);
        softmax_ds(it, bcur, mask_tag);
        if constexpr (BIAS) {
            issue(min(it + 1, total - 1), bcur ^ 1);
            load_bias(min(it + 1, total - 1));
        }
        dkdv_acc(bcur);
        bcur ^= 1;
    };
    int it = 0;
    for (int g = 0; g < p.group; ++g) {
        for (; it < g * nq + (nq - n_mask); ++it) iter(it, std::false_type{});
        if (CAUSAL)
            for (; it < (g + 1) * nq; ++it) iter(it, std::true_type{});
    }

    // ---- merge: waves 4-7 add their dK, dV into waves 0-3's ----
    sync_tiles();  // no copy in flight, every wave done with the tiles and K / V
    float* mg = reinterpret_cast<float*>(smem);
    constexpr int NV = (D / 32) * 16;
    if (st == 1) {
#pragma unroll
        for (int i = 0; i < D / 32; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                mg[(kb * 2 * NV + 16 * i + r) * 64 + lane] = dk[i][r];
                mg[(kb * 2 * NV + NV + 16 * i + r) * 64 + lane] = dv[i][r];
            }
    }
    lds_barrier();
    if (st == 0) {
#pragma unroll
        for (int i = 0; i < D / 32; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                dk[i][r] += mg[(kb * 2 * NV + 16 * i + r) * 64 + lane];
                dv[i][r] += mg[(kb * 2 * NV + NV + 16 * i + r) * 64 + lane];
            }
    }

    // ---- epilogue (waves 0-3): stage dK^T, dV^T through LDS as rows, coalesced stores ----
    constexpr int OW = C::OW;
    constexpr int EPC = 16 / sizeof(T);
    constexpr int CPR = D / EPC;
    T* Os = reinterpret_cast<T*>(smem) + kb * 32 * OW;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        lds_barrier();  // the merge reads / the previous pass's stores are done
        const f32x16* acc = pass == 0 ? dk : dv;
        const float mul = pass == 0 ? p.scale : 1.f;
        if (st == 0) {
#pragma unroll
            for (int i = 0; i < D / 32; ++i)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    s16x4 v4;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v4[e] = Elem<T>::pack1(acc[i][4 * g + e] * mul);
                    *reinterpret_cast<s16x4*>(Os + l32 * OW + 32 * i + 8 * g + 4 * hi) = v4;
                }
        }
        lds_barrier();
        if (st == 0) {
            T* gbase = pass == 0 ? (T*)p.dk + b * p.dk_sb + hk * p.dk_sh : (T*)p.dv + b * p.dv_sb + hk * p.dv_sh;
            const int64_t gss = pass == 0 ? p.dk_ss : p.dv_ss;
#pragma unroll
            for (int i = 0; i < 32 * CPR / 64; ++i) {
                const int cidx = lane + 64 * i;
                const int row = cidx / CPR, col = cidx % CPR;
                const int key = kw0 + row;
                if (key < p.Sk)
                    *reinterpret_cast<uint4*>(gbase + (int64_t)key * gss + col * EPC) =
                        *reinterpret_cast<const uint4*>(Os + row * OW + col * EPC);
            }
        }
    }
}

template <typename T, int D, bool CAUSAL, typename TB>
__global__ __launch_bounds__(512, 1) void dkdv8_kernel(const BwdParams p, const int n_ktiles) {
    __shared__ __attribute__((aligned(16))) char smem[Dkdv8Cfg<T, D>::SMEM_BYTES];
    dkdv8_body<T, D, CAUSAL, TB>(p, n_ktiles, (int)blockIdx.x, (int)gridDim.x, smem);
}


// ---------------------------------------------------------------------------
template <typename T, int D>
struct DqCfg {
    static constexpr bool F32 = Elem<T>::kF32;
    static constexpr int NW = 4;
    static constexpr int NT = 64 * NW;
    static constexpr int BM = 32 * NW;            // queries per workgroup
    static constexpr int NSUB = 2;                // 32-key sub-tiles per tile
    static constexpr int BN = 32 * NSUB;          // keys per tile
    // K / V row stride: conflict-free ds_read_b128 row reads and (16-bit)
    // ds_read_b64_tr_b16 reads of K^T, as for the dK/dV tiles
    static constexpr int KW = D + (F32 ? 4 : (D == 64 ? 8 : 24));
    // K (waves 0-1) and V (waves 2-3) tiles are copied global -> LDS directly
    using Rows = DmaRowGroups<T, BN, D, KW, NW / 2>;
    static constexpr int KALLOC = BN * KW * (int)sizeof(T);
    static constexpr int BUF_BYTES = 2 * KALLOC;    // K rows, V rows
    static constexpr int NBUF = 2;
    static constexpr int OW = D + (F32 ? 4 : 8);
    static constexpr int STAGE_BYTES = NW * 32 * OW * (int)sizeof(T);
    static constexpr int SMEM_BYTES = NBUF * BUF_BYTES > STAGE_BYTES ? NBUF * BUF_BYTES : STAGE_BYTES;
    // fp32 at D=128 needs more than 256 registers per lane (Q, dO and dQ^T in fp32)
    static constexpr int MIN_BLOCKS = ((F32 && D == 128) || D > 128) ? 1 : 2;
};

// KS: key split, as in fwd_kernel: KS groups of 4 waves on the same 128
// queries, group sp walking key tiles sp, sp + KS, ... through its own LDS
// buffers; their dQ partials are summed through LDS at the end (small grids).
// (bid, nblocks: this workgroup among the dQ ones; smem: KS * DqCfg::SMEM_BYTES of LDS)
template <typename T, int D, bool CAUSAL, int DROPOUT, typename TB, int KS>
__device__ FA_INLINE inline void dq_body(const BwdParams& p, const int n_qtiles, const int bid, const int nblocks,
                                        char* smem) {
    using C = DqCfg<T, D>;
    constexpr bool BIAS = !std::is_void<TB>::value;
    using BT = typename std::conditional<BIAS, TB, T>::type;
    using BT16 = typename std::conditional<C::F32, bf16, T>::type;  // the 16-bit input type
    constexpr int BN = C::BN, KW = C::KW;

    const int tid = threadIdx.x;
    // wave index as a scalar: loop bounds derived from it stay wave-uniform
    const int lane = tid & 63, wg = __builtin_amdgcn_readfirstlane(tid >> 6), l32 = lane & 31, hi = lane >> 5;
    // w: the wave's 32-query block, sp: its key split (compile-time 0 without one)
    const int w = KS == 1 ? wg : wg & 3, sp = KS == 1 ? 0 : wg >> 2;
    const int2 tord = tile_order<32 * (KS == 1 ? DqCfg<T, D>::MIN_BLOCKS : 1), CAUSAL>(n_qtiles, bid, nblocks);
    const int qt = n_qtiles - 1 - tord.y;  // longest causal rows first
    const int2 sbh = slice_bh(tord.x, p.H, p.B, !std::is_void<TB>::value && p.bias_sb == 0);
    const int h = sbh.y, b = sbh.x;
    const int hk = h / p.group;
    const int q0 = qt * C::BM;
    const int qw0 = q0 + 32 * w;
    const int qi = qw0 + l32;

    constexpr int QR = C::F32 ? D / 8 : D / 16;
    const bool own_delta = !C::F32 && p.dq_delta;
    uint4 qreg[QR], doreg[QR], oreg[C::F32 ? 1 : QR];
    {
        const T* qrow = (const T*)p.q + b * p.q_sb + (int64_t)qi * p.q_ss + h * p.q_sh;
        const T* drow = (const T*)p.dout + b * p.do_sb + (int64_t)qi * p.do_ss + h * p.do_sh;
        const T* orow = (const T*)p.o + b * p.o_sb + (int64_t)qi * p.o_ss + h * p.o_sh;
#pragma unroll
        for (int i = 0; i < QR; ++i) {
            const int d0 = C::F32 ? hi * (D / 2) + 4 * i : 16 * i + 8 * hi;
            const bool ok = qi < p.Sq;
            qreg[i] = ok ? *reinterpret_cast<const uint4*>(qrow + d0) : make_uint4(0u, 0u, 0u, 0u);
            doreg[i] = ok ? *reinterpret_cast<const uint4*>(drow + d0) : make_uint4(0u, 0u, 0u, 0u);
        }
        if constexpr (!C::F32) {
            if (own_delta) {
#pragma unroll
                for (int i = 0; i < QR; ++i)
                    oreg[i] = qi < p.Sq ? *reinterpret_cast<const uint4*>(orow + 16 * i + 8 * hi)
                                        : make_uint4(0u, 0u, 0u, 0u);
            }
        }
    }
    const int64_t wi = ((int64_t)b * p.H + h) * p.ws_stride + qi;  // qi < sq_pad
    float lse2 = 0.f, del = 0.f, lse_in = 0.f;
    if (own_delta)
        lse_in = qi < p.Sq ? p.lse[((int64_t)b * p.H + h) * p.Sq + qi] : -INFINITY;
    else {
        lse2 = p.lse2[wi];
        del = p.delta[wi];
    }
    // no wait here: these loads stay in flight while the first tile copy is
    // issued (the loop's first barrier waits for both)
    const float c = p.scale_log2;
    uint64_t row_ctr = 0;
    if (DROPOUT) row_ctr = p.offset + ((uint64_t)(b * p.H + h) * (uint64_t)p.Sq + (uint64_t)qi) * (uint64_t)p.Sk;

    f32x16 dq[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) dq[i] = f32x16{};

    int kv_end = p.Sk;
    if (CAUSAL) kv_end = min(kv_end, min(q0 + C::BM, p.Sq));
    const int n_tiles = (kv_end + BN - 1) / BN;
    int n_plain = min(n_tiles, p.Sk / BN);
    if (CAUSAL) n_plain = min(n_plain, (q0 + 1) / BN);
    // this split's local tile j is key tile j * KS + sp; lc(n) counts its
    // local tiles among the first n
    auto lc = [&](int n) { return n > sp ? (n - sp + KS - 1) / KS : 0; };
    const int n_iter = (n_tiles + KS - 1) / KS;
    const int n_tl = lc(n_tiles);
    n_plain = lc(n_plain);

    // ---- K / V tiles: waves 0-1 copy K, waves 2-3 copy V, global -> LDS ----
    const T* kbase = (const T*)p.k + b * p.k_sb + hk * p.k_sh;
    const T* vbase = (const T*)p.v + b * p.v_sb + hk * p.v_sh;
    const bool copy_k = w < C::NW / 2;
    typename C::Rows rows;
    rows.init(copy_k ? p.k_ss : p.v_ss, lane, w % (C::NW / 2));
    auto buf = [&](int s) -> char* { return smem + sp * C::SMEM_BYTES + s * C::BUF_BYTES; };
    auto issue = [&](int j, int s) FA_INLINE {
        const int k0 = (j * KS + sp) * BN;
        const T* src = copy_k ? kbase + (int64_t)k0 * p.k_ss : vbase + (int64_t)k0 * p.v_ss;
        // copies the compiler does not track: it would otherwise make the
        // next LDS read of the current tile wait for them (sync_tiles waits)
        rows.load_untracked(src, copy_k ? p.k_ss : p.v_ss, p.Sk - k0, (const T*)(buf(s) + (copy_k ? 0 : C::KALLOC)));
    };
    // direct-to-LDS copies complete when the issuing wave's vmcnt drains
    auto sync_tiles = [&]() {
        wait_vmem();
        lds_barrier();
    };

    // Two LDS buffers alternate: tile j (64 keys, consumed as two 32-key
    // sub-steps) is read from buffer j&1 while tile j+1 is copied into the
    // other buffer, last read in iteration j-1, which every wave finished
    // before the opening barrier.  Past the last tile the copy repeats it
    // (never read), so the copy is branch-free.
    int bcur = 0;
    if (n_tl > 0) issue(0, 0);

    if constexpr (!C::F32) {
        if (own_delta) {
            // no pre-pass: delta = rowsum(dO * O) of this lane's query from its
            // half of the row (16-byte chunks 2 i + hi) plus the other half in
            // lane l ^ 32, summed in the order delta_kernel sums the row's
            // chunks (chunk sums, then a pairwise tree), so both give the same
            // bits; the rows go to the workspace for the dK/dV pass, which runs
            // after this one.  Rows past Sq: delta = 0, LSE * log2 e = +inf.
            float cs[QR];
#pragma unroll
            for (int i = 0; i < QR; ++i) {
                const s16x8 a = __builtin_bit_cast(s16x8, oreg[i]), d = __builtin_bit_cast(s16x8, doreg[i]);
                float acc = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc += Elem<BT16>::unpack1(a[e]) * Elem<BT16>::unpack1(d[e]);
                cs[i] = acc;
            }
#pragma unroll
            for (int st = QR / 2; st > 0; st >>= 1)
#pragma unroll
                for (int i = 0; i < st; ++i) cs[i] = cs[i] + cs[i + st];
            del = pair_sum(cs[0]);
            lse2 = lse_in == -INFINITY ? INFINITY : lse_in * kLog2e;
            if (sp == 0 && hi == 0) {
                p.lse2[wi] = lse2;
                p.delta[wi] = del;
            }
        }
    }

    // bias of this lane's query row (rows past Sq read zeros, keys past Sk read
    // zeros or the next row: both masked)
    const __amdgpu_buffer_rsrc_t brs =
        slice_buffer((const BT*)p.bias + b * p.bias_sb + h * p.bias_sh, BIAS ? p.bias_span : 0);
    const int bvoff = (qi * (int)p.bias_ss + 4 * hi) * (int)sizeof(BT);

    // one 32-key sub-step of the tile in buffer `bcur` starting at key k0
    auto sub = [&](int k0, const T* Ks, const T* Vs, auto mask_tag) FA_INLINE {
        constexpr bool MASK = decltype(mask_tag)::value;
        constexpr int BN = 32;
        const bool active = !MASK || !CAUSAL || k0 <= qw0 + 31;
        if (active) {
            // bias of keys {8 g + 4 hi + 0..3}
            bias4_t<BT> bv[BIAS ? 4 : 1];
            if constexpr (BIAS) {
                // tiles of plain steps are whole
                auto load_all = [&](auto full_tag) FA_INLINE {
#pragma unroll
                    for (int g = 0; g < 4; ++g)
                        bv[g] = load_bias4<BT, decltype(full_tag)::value>(brs, bvoff, (k0 + 8 * g) * (int)sizeof(BT));
                };
                if (!MASK || k0 + BN <= p.Sk)
                    load_all(std::true_type{});
                else
                    load_all(std::false_type{});
            }
            // the forward's keep bits of this lane's query for the sub-step's keys
            uint32_t kword = 0;
            if (DROPOUT == 2 && qi < p.Sq && k0 < p.Sk)
                kword = p.kb[((int64_t)(b * p.H + h) * p.Sq + qi) * p.kb_w + (k0 >> 5)];
            // ---- S^T = K Q^T, dP^T = V dO^T (C[key][query]) ----
            f32x16 s = f32x16{}, dp = f32x16{};
            const T* krow = Ks + l32 * KW;
            const T* vrow = Vs + l32 * KW;
            if constexpr (C::F32) {
#pragma unroll
                for (int i = 0; i < QR; ++i) {
                    const f32x4 ak = *reinterpret_cast<const f32x4*>(krow + hi * (D / 2) + 4 * i);
                    const f32x4 av = *reinterpret_cast<const f32x4*>(vrow + hi * (D / 2) + 4 * i);
                    const f32x4 bq = __builtin_bit_cast(f32x4, qreg[i]);
                    const f32x4 bd = __builtin_bit_cast(f32x4, doreg[i]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        s = mfma_f32(ak[e], bq[e], s);
                        dp = mfma_f32(av[e], bd[e], dp);
                    }
                }
            } else {
#pragma unroll
                for (int kk = 0; kk < QR; ++kk) {
                    const s16x8 ak = *reinterpret_cast<const s16x8*>(krow + 16 * kk + 8 * hi);
                    const s16x8 av = *reinterpret_cast<const s16x8*>(vrow + 16 * kk + 8 * hi);
                    s = Elem<T>::mfma(ak, __builtin_bit_cast(s16x8, qreg[kk]), s);
                    dp = Elem<T>::mfma(av, __builtin_bit_cast(s16x8, doreg[kk]), dp);
                }
            }
            // ---- dS^T = P^T (dP^T - delta); scale applied at the end ----
            const bool need_mask = MASK && ((k0 + BN > p.Sk) || (CAUSAL && k0 + BN - 1 > qw0));
            // key k0 + 4 hi + o (o = 8 (r / 4) + r % 4) is masked when it is >= Sk
            // or (causal) > qi: one per-lane bound against constants
            const int lim = (CAUSAL ? min(p.Sk, qi + 1) : p.Sk) - k0 - 4 * hi;
            // stored keep bits: key k0 + 8 g + 4 hi + e at bit 8 g + e after the shift
            const uint32_t km = DROPOUT == 2 ? kword >> (4 * hi) : 0u;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + 8 * (r >> 2) + 4 * hi + (r & 3);
                float pv;
                if constexpr (BIAS)
                    pv = fast_exp2(__builtin_fmaf(s[r], c, __builtin_fmaf(bias_f32<BT>(bv[r >> 2][r & 3]), kLog2e, -lse2)));
                else
                    pv = fast_exp2(__builtin_fmaf(s[r], c, -lse2));
                if (need_mask && 8 * (r >> 2) + (r & 3) >= lim) pv = 0.f;
                if (DROPOUT) {
                    const uint32_t m = DROPOUT == 2 ? bit_mask(km, 8 * (r >> 2) + (r & 3))
                                       : (philox_keep(p.seed, row_ctr + (uint64_t)key, p.keep_thresh) ? ~0u : 0u);
                    s[r] = pv * __builtin_fmaf(keep_or_zero(dp[r], m), p.rp, -del);
                } else {
                    s[r] = pv * (dp[r] - del);
                }
            }
            // ---- dQ^T += K^T dS^T ----
            if constexpr (C::F32) {
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    const T* kr = Ks + (8 * (t >> 2) + 4 * hi + (t & 3)) * KW + l32;
#pragma unroll
                    for (int i = 0; i < D / 32; ++i) dq[i] = mfma_f32(kr[32 * i], s[t], dq[i]);
                }
            } else {
                // K^T operand straight from the row-major K tile: lane (d, h)
                // takes keys 16 ks + {4h .. 4h+3, 8+4h .. 8+4h+3}, the keys of
                // its dS^T values
                const int trow = 4 * hi + ((lane & 15) >> 2);
                const int tcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
                for (int ks = 0; ks < BN / 16; ++ks) {
                    float ts[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) ts[e] = s[8 * ks + e];
                    const s16x8 bs8 = pack8<T>(ts);
#pragma unroll
                    for (int i = 0; i < D / 32; ++i) {
                        const T* kp = Ks + (16 * ks + trow) * KW + 32 * i + tcol;
                        const s16x8 a = cat4(lds_read_tr16(kp), lds_read_tr16(kp + 8 * KW));
                        dq[i] = Elem<T>::mfma(a, bs8, dq[i]);
                    }
                }
            }
        }
    };
    // 16-bit inputs without bias or dropout: the S / dP products of a tile's
    // two sub-steps are issued before the dS of either, so the dS arithmetic of
    // the first overlaps the products of the second inside the wave (the same
    // arithmetic in the same order as `sub`, so the same bits)
    constexpr bool PIPE = !C::F32 && !BIAS && DROPOUT == 0;
    using TP = BT16;  // T for the 16-bit inputs these two serve
    auto sdp16 = [&](const T* Ks, const T* Vs, f32x16& s, f32x16& dp) FA_INLINE {
        s = f32x16{};
        dp = f32x16{};
        const T* krow = Ks + l32 * KW;
        const T* vrow = Vs + l32 * KW;
#pragma unroll
        for (int kk = 0; kk < QR; ++kk) {
            const s16x8 ak = *reinterpret_cast<const s16x8*>(krow + 16 * kk + 8 * hi);
            const s16x8 av = *reinterpret_cast<const s16x8*>(vrow + 16 * kk + 8 * hi);
            s = Elem<TP>::mfma(ak, __builtin_bit_cast(s16x8, qreg[kk]), s);
            dp = Elem<TP>::mfma(av, __builtin_bit_cast(s16x8, doreg[kk]), dp);
        }
    };
    auto fin16 = [&](int k0, const T* Ks, f32x16& s, const f32x16& dp, auto mask_tag) FA_INLINE {
        constexpr bool MASK = decltype(mask_tag)::value;
        const bool need_mask = MASK && ((k0 + 32 > p.Sk) || (CAUSAL && k0 + 31 > qw0));
        const int lim = (CAUSAL ? min(p.Sk, qi + 1) : p.Sk) - k0 - 4 * hi;  // as in `sub`
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float pv = fast_exp2(__builtin_fmaf(s[r], c, -lse2));
            if (need_mask && 8 * (r >> 2) + (r & 3) >= lim) pv = 0.f;
            s[r] = pv * (dp[r] - del);
        }
        const int trow = 4 * hi + ((lane & 15) >> 2);
        const int tcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            float ts[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) ts[e] = s[8 * ks + e];
            const s16x8 bs8 = pack8<TP>(ts);
#pragma unroll
            for (int i = 0; i < D / 32; ++i) {
                const T* kp = Ks + (16 * ks + trow) * KW + 32 * i + tcol;
                const s16x8 a = cat4(lds_read_tr16(kp), lds_read_tr16(kp + 8 * KW));
                dq[i] = Elem<TP>::mfma(a, bs8, dq[i]);
            }
        }
    };
    auto step = [&](int j, auto mask_tag) FA_INLINE {
        sync_tiles();
        issue(min(j + 1, n_tl - 1), bcur ^ 1);
        if constexpr (PIPE) {
            static_assert(C::NSUB == 2, "two sub-steps per tile");
            constexpr bool MASK = decltype(mask_tag)::value;
            const int ka = (j * KS + sp) * C::BN, kb2 = ka + 32;
            const T* ksa = (const T*)buf(bcur);
            const T* vsa = (const T*)(buf(bcur) + C::KALLOC);
            const bool act_a = !MASK || !CAUSAL || ka <= qw0 + 31;
            const bool act_b = !MASK || !CAUSAL || kb2 <= qw0 + 31;
            f32x16 sa, dpa, sb, dpb;
            if (act_a) sdp16(ksa, vsa, sa, dpa);
            if (act_b) sdp16(ksa + 32 * KW, vsa + 32 * KW, sb, dpb);
            if (act_a) fin16(ka, ksa, sa, dpa, mask_tag);
            if (act_b) fin16(kb2, ksa + 32 * KW, sb, dpb, mask_tag);
        } else {
#pragma unroll
            for (int st = 0; st < C::NSUB; ++st)
                sub((j * KS + sp) * C::BN + 32 * st, (const T*)buf(bcur) + 32 * st * KW,
                    (const T*)(buf(bcur) + C::KALLOC) + 32 * st * KW, mask_tag);
        }
        bcur ^= 1;
    };

    for (int j = 0; j < n_plain; ++j) step(j, std::false_type{});
    for (int j = n_plain; j < n_tl; ++j) step(j, std::true_type{});
    // splits with fewer tiles pass the barriers of the others' last iteration
    for (int j = n_tl; j < n_iter; ++j) sync_tiles();

    sync_tiles();  // no copy in flight, all waves done with the tiles
    if constexpr (KS > 1) {
        // ---- sum the splits' dQ into split 0 through LDS ----
        constexpr int NO = (D / 32) * 16;
        static_assert((KS - 1) * 4 * NO * 64 * 4 <= (KS - 1) * C::SMEM_BYTES, "parts fit the other splits' buffers");
        float* mg = reinterpret_cast<float*>(smem + C::SMEM_BYTES);
        auto at = [&](int s2, int f) FA_INLINE { return mg + (((s2 - 1) * 4 + w) * NO + f) * 64 + lane; };
        if (sp > 0) {
#pragma unroll
            for (int i = 0; i < D / 32; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) *at(sp, 16 * i + r) = dq[i][r];
        }
        lds_barrier();
        if (sp == 0) {
#pragma unroll
            for (int s2 = 1; s2 < KS; ++s2)
#pragma unroll
                for (int i = 0; i < D / 32; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) dq[i][r] += *at(s2, 16 * i + r);
        }
    }
    // ---- epilogue (split 0): stage dQ^T through LDS as rows, coalesced stores ----
    constexpr int OW = C::OW;
    T* Os = (T*)smem + w * 32 * OW;
    if (sp == 0) {
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * i + 8 * g + 4 * hi;
            if constexpr (C::F32) {
                f32x4 v4;
#pragma unroll
                for (int e = 0; e < 4; ++e) v4[e] = dq[i][4 * g + e] * p.scale;
                *reinterpret_cast<f32x4*>(Os + l32 * OW + d) = v4;
            } else {
                s16x4 v4;
#pragma unroll
                for (int e = 0; e < 4; ++e) v4[e] = Elem<T>::pack1(dq[i][4 * g + e] * p.scale);
                *reinterpret_cast<s16x4*>(Os + l32 * OW + d) = v4;
            }
        }
    }
    lds_barrier();
    constexpr int EPC = 16 / sizeof(T);
    constexpr int CPR = D / EPC;
    T* gbase = (T*)p.dq + b * p.dq_sb + h * p.dq_sh;
    if (sp == 0) {
#pragma unroll
        for (int i = 0; i < 32 * CPR / 64; ++i) {
            const int cidx = lane + 64 * i;
            const int row = cidx / CPR, col = cidx % CPR;
            const int q = qw0 + row;
            if (q < p.Sq)
                *reinterpret_cast<uint4*>(gbase + (int64_t)q * p.dq_ss + col * EPC) =
                    *reinterpret_cast<const uint4*>(Os + row * OW + col * EPC);
        }
    }
}

template <typename T, int D, bool CAUSAL, int DROPOUT, typename TB, int KS>
__global__ __launch_bounds__(256 * KS, (KS == 1 ? DqCfg<T, D>::MIN_BLOCKS : 1)) void dq_kernel(const BwdParams p,
                                                                                           const int n_qtiles) {
    __shared__ __attribute__((aligned(16))) char smem[DqCfg<T, D>::SMEM_BYTES * KS];
    dq_body<T, D, CAUSAL, DROPOUT, TB, KS>(p, n_qtiles, (int)blockIdx.x, (int)gridDim.x, smem);
}

// ---------------------------------------------------------------------------
// A whole backward on a grid smaller than the CU count (16-bit inputs, D = 64
// or 128, no bias or dropout), after the delta pre-pass: the dK/dV workgroups
// (dkdv8_body) and the key-split dQ workgroups (dq_body, KS = 2) of the two
// passes in one launch, interleaved longest first.  Each pass alone leaves CUs
// idle and runs for the length of its longest workgroup's tile chain; together
// they share the CUs and the two chains overlap.  Per element the arithmetic
// is that of the two kernels (and of dq_kernel after the pre-pass), so the
// outputs are bit-identical to running them one after the other.
template <typename T, int D>
struct BwdSmallCfg {
    static constexpr int S1 = Dkdv8Cfg<T, D>::SMEM_BYTES, S2 = 2 * DqCfg<T, D>::SMEM_BYTES;
    static constexpr int SMEM_BYTES = S1 > S2 ? S1 : S2;
    static_assert(Dkdv8Cfg<T, D>::NT == 512 && 2 * DqCfg<T, D>::NT == 512, "one workgroup size");
    static_assert(SMEM_BYTES <= 160 * 1024, "LDS of one CU");
};

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(512, 1) void bwd_small_kernel(const BwdParams p, const int n_ktiles, const int n_kv,
                                                          const int n_qtiles, const int n_q) {
    __shared__ __attribute__((aligned(16))) char smem[BwdSmallCfg<T, D>::SMEM_BYTES];
    // workgroups 2 i and 2 i + 1 take the i-th dK/dV and dQ ones while both
    // kinds last, then the rest of the larger kind
    const int b = (int)blockIdx.x;
    const int m = min(n_kv, n_q);
    bool kv;
    int idx;
    if (b < 2 * m) {
        kv = (b & 1) == 0;
        idx = b >> 1;
    } else {
        kv = n_kv > n_q;
        idx = m + (b - 2 * m);
    }
    if (kv)
        dkdv8_body<T, D, CAUSAL, void>(p, n_ktiles, idx, n_kv, smem);
    else
        dq_body<T, D, CAUSAL, 0, void, 2>(p, n_qtiles, idx, n_q, smem);
}


// ---------------------------------------------------------------------------
// Ping-pong dQ for 16-bit inputs without bias or dropout, D = 128, on grids
// that fill the CUs.  One workgroup = 8 waves = 256 queries of one (batch,
// head), one workgroup per CU, like the ping-pong forward: waves w and w + 4
// share a SIMD and own the adjacent 32-query blocks 2 (w % 4) and 2 (w % 4) + 1
// (similar causal lengths); Q, dO (and O, for delta) of the wave's queries sit
// in registers.  64-key tiles of K and V rotate through four LDS slots.  Every
// wave runs, for each key tile r,
//   M(r): dQ^T += K(r-1)^T dS^T(r-1), then S^T(r) = K Q^T, dP^T(r) = V dO^T
//   V(r): P = exp2(S c - LSE), dS = P (dP - delta), packed to 16 bits
// with a workgroup barrier after each phase; waves 4-7 run one phase behind,
// so one wave's 48 matrix products overlap the other's arithmetic.  The tile
// copies (direct to LDS) go in the V phases: waves 0-3 copy K(r + 2), waves
// 4-7 V(r + 3) in round r (4 or 5 copy instructions each); a slot is refilled
// only after both groups' M phases that read its previous tile, and a wave's
// copies have landed before the barrier that opens the first M phase reading
// them (modelled for every run length up to 100 tiles by
// tests/test_pp_schedule_cpu.py).
// Per query the arithmetic is that of dq_kernel, in the same order (delta and
// LSE * log2 e computed as there and written to the workspace rows for the
// dK/dV pass), so dQ and the workspace rows are bit-identical to it.
template <typename T, int D>
struct DqPPCfg {
    static constexpr int NW = 8;
    static constexpr int NT = 64 * NW;
    static constexpr int BM = 32 * NW;               // queries per workgroup
    static constexpr int BN = 64;                    // keys per tile
    static constexpr int KW = D + 24;                // K / V row stride, as in dq_kernel
    static constexpr int KALLOC = BN * KW * (int)sizeof(T);
    static constexpr int SLOT_BYTES = 2 * KALLOC;    // K rows, V rows
    static constexpr int NSLOT = 4;
    static constexpr int SMEM_BYTES = NSLOT * SLOT_BYTES;
    static constexpr int EPC = 16 / (int)sizeof(T);
    static constexpr int CW = KW / EPC;              // 16-byte chunks per LDS row
    static constexpr int NI = BN * CW / 64;          // copy instructions per tile and matrix
    static_assert((BN * CW) % 64 == 0, "whole copy instructions");
    static constexpr int PER = (NI + 3) / 4;         // per wave of a group (at most)
    static constexpr int OW = D + 8;                 // output staging row stride
    static_assert(SMEM_BYTES <= 160 * 1024, "LDS of one CU");
    static_assert(NW * 32 * OW * (int)sizeof(T) <= SMEM_BYTES, "output staging");
};

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(512, 1) void dq_pp_kernel(const BwdParams p) {
    using C = DqPPCfg<T, D>;
    static_assert(!Elem<T>::kF32 && D == 128, "16-bit inputs, D = 128");
    constexpr int BN = C::BN, KW = C::KW, NSLOT = C::NSLOT;
    __shared__ __attribute__((aligned(16))) char smem[C::SMEM_BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), l32 = lane & 31, hi = lane >> 5;
    const int grp = w >> 2, w4 = w & 3;
    const int blk = 2 * w4 + grp;
    const int n_qtiles = (p.Sq + C::BM - 1) / C::BM;
    const int2 tord = tile_order<32, CAUSAL>(n_qtiles);
    const int bh = tord.x;
    const int qt = n_qtiles - 1 - tord.y;  // longest causal rows first
    const int h = bh % p.H, b = bh / p.H;
    const int hk = h / p.group;
    const int q0 = qt * C::BM;
    const int qw0 = q0 + 32 * blk;
    const int qi = qw0 + l32;

    // ---- Q, dO (and O) rows of this lane's query in registers (MFMA B operands) ----
    // Branch-free buffer loads over the workgroup's rows [q0, min(Sq, q0 + BM)):
    // rows past Sq read zeros (out of the descriptor's range).  All of the
    // prologue's loads and copies are issued before its one wait (conditional
    // loads made the compiler wait between them: several memory round trips
    // per workgroup, exposed at one workgroup per CU).
    constexpr int QR = D / 16;
    const bool own_delta = p.dq_delta != 0;
    const int qrows = min(p.Sq - q0, C::BM);  // >= 1: q0 < Sq
    auto rows_rsrc = [&](const void* base, int64_t ss) FA_INLINE {
        return slice_buffer((const T*)base + (int64_t)q0 * ss, ((qrows - 1) * (int)ss + D) * (int)sizeof(T));
    };
    const int rrow = 32 * blk + l32;  // this lane's row in the block
    uint4 qreg[QR], doreg[QR], oreg[QR];
    {
        const __amdgpu_buffer_rsrc_t rq = rows_rsrc((const T*)p.q + b * p.q_sb + h * p.q_sh, p.q_ss);
        const __amdgpu_buffer_rsrc_t rd = rows_rsrc((const T*)p.dout + b * p.do_sb + h * p.do_sh, p.do_ss);
#pragma unroll
        for (int i = 0; i < QR; ++i) {
            const int d0 = 16 * i + 8 * hi;
            qreg[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    rq, (rrow * (int)p.q_ss + d0) * (int)sizeof(T), 0, 0));
            doreg[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                     rd, (rrow * (int)p.do_ss + d0) * (int)sizeof(T), 0, 0));
        }
        if (own_delta) {
            const __amdgpu_buffer_rsrc_t ro = rows_rsrc((const T*)p.o + b * p.o_sb + h * p.o_sh, p.o_ss);
#pragma unroll
            for (int i = 0; i < QR; ++i)
                oreg[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        ro, (rrow * (int)p.o_ss + 16 * i + 8 * hi) * (int)sizeof(T), 0, 0));
        }
    }
    // the workspace rows hold sq_pad (Sq rounded up to 128) entries; the last
    // 256-query block may reach past them (its queries past Sq get P = 0)
    const bool in_ws = qi < p.sq_pad;
    const int64_t wi = ((int64_t)b * p.H + h) * p.ws_stride + qi;
    // the saved LSE (own_delta) or the workspace rows (after a delta pre-pass):
    // both loaded without a branch, used after the tile copies are issued
    // (rows past Sq / sq_pad read zeros and are replaced then)
    const __amdgpu_buffer_rsrc_t rl = slice_buffer(p.lse + ((int64_t)b * p.H + h) * p.Sq, own_delta ? p.Sq * 4 : 0);
    const __amdgpu_buffer_rsrc_t rw =
        slice_buffer(p.lse2 + ((int64_t)b * p.H + h) * p.ws_stride, own_delta ? 0 : p.ws_stride * 4);
    const float lse_raw = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rl, qi * 4, 0, 0));
    const float ws_lse = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rw, qi * 4, 0, 0));
    const float ws_del = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rw, (p.sq_pad + qi) * 4, 0, 0));
    float lse2 = INFINITY, del = 0.f;
    const float c = p.scale_log2;
    f32x16 dq[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) dq[i] = f32x16{};

    int kv_end = p.Sk;
    if (CAUSAL) kv_end = min(kv_end, min(q0 + C::BM, p.Sq));
    const int n_tiles = (kv_end + BN - 1) / BN;
    // key tiles this wave uses, and how many of them need no mask
    int n_w = qw0 < p.Sq ? n_tiles : 0;
    if (CAUSAL) n_w = min(n_w, (qw0 + 31) / BN + 1);
    int n_um = min(n_w, p.Sk / BN);
    if (CAUSAL) n_um = min(n_um, (qw0 + 1) / BN);

    // ---- K / V tile copies: waves 0-3 K, waves 4-7 V (instructions w4, w4 + 4, ...) ----
    auto opaque64 = [](uint64_t x) FA_INLINE {
        asm volatile("" : "+s"(x));
        return x;
    };
    auto opaque32 = [](uint32_t x) FA_INLINE {
        asm volatile("" : "+s"(x));
        return x;
    };
    const int64_t css = grp == 0 ? p.k_ss : p.v_ss;
    const uint64_t cbase = opaque64((uint64_t)(uintptr_t)(grp == 0 ? (const T*)p.k + b * p.k_sb + hk * p.k_sh
                                                                   : (const T*)p.v + b * p.v_sb + hk * p.v_sh));
    const uint64_t crow = opaque64((uint64_t)css * sizeof(T));
    const uint32_t full_bytes = (uint32_t)(((BN - 1) * (int)css + D) * (int)sizeof(T));
    const int n_copy = (C::NI - w4 + 3) / 4;  // this wave's instructions per tile (wave-uniform)
    int coff[C::PER];
#pragma unroll
    for (int t = 0; t < C::PER; ++t) {
        const int cidx = 64 * (w4 + 4 * t) + lane;
        const int row = cidx / C::CW, col = cidx % C::CW;
        // padding chunks of an LDS row read nothing (out of the buffer's range)
        coff[t] = col < D / C::EPC ? (row * (int)css + col * C::EPC) * (int)sizeof(T) : kOffNowhere;
    }
    auto slot = [&](int r) FA_INLINE -> char* { return smem + (r & (NSLOT - 1)) * C::SLOT_BYTES; };
    static_assert(NSLOT == 4, "slot index by mask");
    // tile j < n_tiles at source src, LDS address l0: the keys [j BN, min(Sk, j BN + BN)),
    // rows past Sk land as zeros (only the last tile can be partial)
    const uint32_t last_bytes = opaque32(
        p.Sk - (n_tiles - 1) * BN >= BN ? full_bytes
                                        : (uint32_t)(((p.Sk - (n_tiles - 1) * BN - 1) * (int)css + D) * (int)sizeof(T)));
    auto issue_at = [&](int j, uint64_t src, uint32_t l0) FA_INLINE {
        u32x4 rs;
        rs[0] = (uint32_t)src;
        rs[1] = (uint32_t)(src >> 32) & 0xFFFFu;
        rs[2] = j == n_tiles - 1 ? last_bytes : full_bytes;
        rs[3] = 0x00020000u;
#pragma unroll
        for (int t = 0; t < C::PER; ++t) {
            const int g = w4 + 4 * t;  // wave-uniform
            if (g < C::NI) dma_load16_untracked(rs, __builtin_amdgcn_readfirstlane(l0 + 1024 * g), coff[t]);
        }
    };
    auto issue = [&](int j) FA_INLINE {
        issue_at(j, cbase + (uint64_t)(int64_t)(j * BN) * crow,
                 __builtin_amdgcn_readfirstlane(lds_addr(slot(j) + grp * C::KALLOC)));
    };
    // the rounds' copy cursor (tile r + 2 + grp): source and LDS slot advanced
    // by additions, no multiplication in the loop
    const uint64_t dsrc = opaque64((uint64_t)BN * crow);
    const uint32_t lds_first = __builtin_amdgcn_readfirstlane(lds_addr(smem + grp * C::KALLOC));
    const uint32_t lds_wrap = lds_first + NSLOT * C::SLOT_BYTES;
    uint64_t kc_src = opaque64(cbase + (uint64_t)(2 + grp) * dsrc);
    uint32_t kc_lds = lds_first + (uint32_t)(((2 + grp) & (NSLOT - 1)) * C::SLOT_BYTES);

    // ---- M phase: dQ^T of the previous tile, then S^T / dP^T of this one ----
    // dQ step t (t = ks (D / 32) + i, ks = 16-key step of the 64): K^T of keys
    // 16 ks + ..., d block i (transposing reads of the K tile); S/dP step
    // t = 2 kk + kb: the K, V row fragments d = 16 kk + 8 hi of key 32 kb + l32.
    const int trow = 4 * hi + ((lane & 15) >> 2);
    const int tcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    constexpr int NA = (BN / 16) * (D / 32);  // dQ steps (one product each)
    constexpr int NB = 2 * QR;                // S/dP steps (an S and a dP product each)
    constexpr int NSTEP = NA + NB;
    constexpr int MP = 3;
    s16x8 bs8[BN / 16];       // dS^T of the previous tile (B operands)
    f32x16 sc[2], dpc[2];     // S^T, dP^T of this tile, per 32-key block
    // the first MP dQ steps' K^T operands of round r, read at the end of the
    // previous V phase (tile r - 1 stays in its slot until round r + 2)
    s16x8 xpre[MP];
    auto prefetch = [&](int r) FA_INLINE {
        const T* Ka = (const T*)slot(r + NSLOT - 1);
#pragma unroll
        for (int t = 0; t < MP; ++t) {
            const int ks = t / (D / 32), i = t % (D / 32);
            const T* kp = Ka + (16 * ks + trow) * KW + 32 * i + tcol;
            xpre[t] = cat4(lds_read_tr16(kp), lds_read_tr16(kp + 8 * KW));
        }
    };
    auto mphase = [&](int r, auto a_tag, auto b_tag) FA_INLINE {
        constexpr bool A = decltype(a_tag)::value, BB = decltype(b_tag)::value;
        const T* Ka = (const T*)slot(r + NSLOT - 1);
        const T* Kb = (const T*)slot(r) + l32 * KW + 8 * hi;
        const T* Vb = (const T*)(slot(r) + C::KALLOC) + l32 * KW + 8 * hi;
        s16x8 x[NSTEP], y[NSTEP];
        auto rd = [&](int t) FA_INLINE {
            if (t < NA) {
                const int ks = t / (D / 32), i = t % (D / 32);
                const T* kp = Ka + (16 * ks + trow) * KW + 32 * i + tcol;
                x[t] = cat4(lds_read_tr16(kp), lds_read_tr16(kp + 8 * KW));
            } else {
                const int u = t - NA, kk = u >> 1, kb = u & 1;
                x[t] = *reinterpret_cast<const s16x8*>(Kb + 32 * kb * KW + 16 * kk);
                y[t] = *reinterpret_cast<const s16x8*>(Vb + 32 * kb * KW + 16 * kk);
            }
        };
        auto mm = [&](int t) FA_INLINE {
            if (t < NA) {
                const int ks = t / (D / 32), i = t % (D / 32);
                dq[i] = Elem<T>::mfma(x[t], bs8[ks], dq[i]);
            } else {
                const int u = t - NA, kk = u >> 1, kb = u & 1;
                sc[kb] = Elem<T>::mfma(x[t], __builtin_bit_cast(s16x8, qreg[kk]), kk == 0 ? f32x16{} : sc[kb]);
                dpc[kb] = Elem<T>::mfma(y[t], __builtin_bit_cast(s16x8, doreg[kk]), kk == 0 ? f32x16{} : dpc[kb]);
            }
        };
        constexpr int T0 = A ? 0 : NA, T1 = BB ? NSTEP : NA;
        static_assert(MP <= NA, "prefetched steps are dQ steps");
#pragma unroll
        for (int t = T0; t < T0 + MP; ++t) {
            if (A)
                x[t] = xpre[t];
            else
                rd(t);
        }
#pragma unroll
        for (int t = T0; t < T1; ++t) {
            if (t + MP < T1) rd(t + MP);
            mm(t);
        }
        // the same order for the scheduler: reads of MP steps, then per step
        // its products followed by the reads of step t + MP
        auto rd_group = [&](int t) FA_INLINE {  // 2 transposing reads, or 2 row reads
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        };
        auto mf_group = [&](int t) FA_INLINE {
            if (t < NA)
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            else
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        };
        if (!A) {
#pragma unroll
            for (int t = T0; t < T0 + MP; ++t) rd_group(t);
        }
#pragma unroll
        for (int t = T0; t < T1; ++t) {
            mf_group(t);
            if (t + MP < T1) rd_group(t + MP);
        }
    };

    // ---- V phase of tile r: dS^T = P^T (dP^T - delta), packed (mask: diagonal / tail tiles) ----
    auto vphase = [&](int r, bool msk) FA_INLINE {
        float ds[2][16];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float pv = fast_exp2(__builtin_fmaf(sc[kb][e], c, -lse2));
                ds[kb][e] = pv * (dpc[kb][e] - del);
            }
        if (msk) {
            // key r BN + 32 kb + 8 g + 4 hi + f (e = 4 g + f) is masked when it
            // is >= Sk or (causal) > qi: one per-lane bound against constants
            const int kbase = r * BN + 4 * hi;
            const int lim = CAUSAL ? min(p.Sk - 1, qi) - kbase : p.Sk - 1 - kbase;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    if (32 * kb + 8 * (e >> 2) + (e & 3) > lim) ds[kb][e] = 0.f;
        }
#pragma unroll
        for (int ks = 0; ks < BN / 16; ++ks) bs8[ks] = pack8<T>(&ds[ks >> 1][8 * (ks & 1)]);
    };

    auto sched_fence = [&]() FA_INLINE { __builtin_amdgcn_sched_barrier(0); };
    using TT = std::true_type;
    using FF = std::false_type;

    // prologue: tiles 0, 1, 2 (every wave its instructions of each)
    for (int j = 0; j < 3; ++j)
        if (j < n_tiles) issue(j);
    if (own_delta) {
        // delta = rowsum(dO * O) as dq_kernel computes it (16-byte chunk sums,
        // then a pairwise tree, then the lane pair), written to the workspace
        // with LSE * log2 e; rows past Sq: delta = 0, LSE * log2 e = +inf
        float cs[QR];
#pragma unroll
        for (int i = 0; i < QR; ++i) {
            const s16x8 a = __builtin_bit_cast(s16x8, oreg[i]), d = __builtin_bit_cast(s16x8, doreg[i]);
            float acc = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc += Elem<T>::unpack1(a[e]) * Elem<T>::unpack1(d[e]);
            cs[i] = acc;
        }
#pragma unroll
        for (int st = QR / 2; st > 0; st >>= 1)
#pragma unroll
            for (int i = 0; i < st; ++i) cs[i] = cs[i] + cs[i + st];
        del = pair_sum(cs[0]);
        const float lse_in = qi < p.Sq ? lse_raw : -INFINITY;
        lse2 = lse_in == -INFINITY ? INFINITY : lse_in * kLog2e;
    } else {
        lse2 = in_ws ? ws_lse : INFINITY;
        del = in_ws ? ws_del : 0.f;
    }
    wait_vmem();
    lds_barrier();
    // the rows go to the workspace for the dK/dV pass (a later launch); issued
    // after the barrier so that no wait of the prologue covers the stores
    if (own_delta && hi == 0 && in_ws) {
        p.lse2[wi] = lse2;
        p.delta[wi] = del;
    }
    if (grp == 1) barrier_no_fence();  // waves 4-7 run one phase behind

    // V phase of round r: this round's copies (tile r + 2 + grp; tiles 0-2 came
    // with the prologue), then dS of tile r (zero where the wave has no tile r),
    // then wait for this wave's copies of earlier rounds
    auto vround = [&](int r) FA_INLINE {
        const int j = r + 2 + grp;
        const bool cp = j >= 3 && j < n_tiles;
        if (cp) issue_at(j, kc_src, kc_lds);
        kc_src += dsrc;
        kc_lds += C::SLOT_BYTES;
        if (kc_lds == lds_wrap) kc_lds = lds_first;
        if (r < n_w)
            vphase(r, r >= n_um);
        else {
#pragma unroll
            for (int ks = 0; ks < BN / 16; ++ks) bs8[ks] = s16x8{};
        }
        if (r + 1 <= n_tiles) prefetch(r + 1);
        if (!cp)
            wait_vmem();
        else if (n_copy == C::PER)
            wait_vmem_below<C::PER>();
        else
            wait_vmem_below<C::PER - 1>();
    };
    // Round 0 runs S/dP only; rounds 1 .. n_tiles run both halves of the M
    // phase unconditionally (one code path keeps the accumulators in place):
    // a wave past its last tile gets dS = 0, and the S/dP products of round
    // n_tiles (no tile) are not used.
    if (n_tiles > 0) {
        sched_fence();
        mphase(0, FF{}, TT{});
        sched_fence();
        barrier_no_fence();
        sched_fence();
        vround(0);
        sched_fence();
        barrier_no_fence();
        for (int r = 1; r <= n_tiles; ++r) {
            sched_fence();
            mphase(r, TT{}, TT{});
            sched_fence();
            barrier_no_fence();
            sched_fence();
            vround(r);
            sched_fence();
            barrier_no_fence();
        }
    }
    if (grp == 0) barrier_no_fence();
    sched_fence();

    // ---- epilogue: stage dQ^T through LDS as rows, coalesced stores ----
    // (every M phase is done: the last barrier follows the last M phase of waves 4-7)
    constexpr int OW = C::OW;
    T* Os = reinterpret_cast<T*>(smem) + w * 32 * OW;
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            s16x4 v4;
#pragma unroll
            for (int e = 0; e < 4; ++e) v4[e] = Elem<T>::pack1(dq[i][4 * g + e] * p.scale);
            *reinterpret_cast<s16x4*>(Os + l32 * OW + 32 * i + 8 * g + 4 * hi) = v4;
        }
    lds_barrier();
    constexpr int EPC = 16 / sizeof(T);
    constexpr int CPR = D / EPC;
    T* gbase = (T*)p.dq + b * p.dq_sb + h * p.dq_sh;
#pragma unroll
    for (int i = 0; i < 32 * CPR / 64; ++i) {
        const int cidx = lane + 64 * i;
        const int row = cidx / CPR, col = cidx % CPR;
        const int q = qw0 + row;
        if (q < p.Sq)
            *reinterpret_cast<uint4*>(gbase + (int64_t)q * p.dq_ss + col * EPC) =
                *reinterpret_cast<const uint4*>(Os + row * OW + col * EPC);
    }
}

// ---------------------------------------------------------------------------
// dQ from the stored dS (16-bit inputs with a bias gradient requested).  The
// dK/dV pass writes dS = P (dP - delta) of every (query, key) it visits into
// the gradient buffer (per batch and head; ES bytes per element: the input
// dtype or float32), which covers every (query, key) this pass reads: a
// key block of 128 visits the queries from its first key on, and a 128-query
// tile here reads keys below its end only under the causal mask.  So dQ =
// scale * dS K is a single product per (batch, head, 128-query tile): dS rows
// and K rows stream global -> LDS, and no S, P or dP is recomputed.
// Causal, with `fill`, the pass also writes the zeros that no kernel visits:
// keys from the tile's end (q0 + 128) on, whole row tails.  (Spreading them
// over the key loop does not overlap them with its reads: the pass is bound
// by the HBM traffic of both.)
template <typename T, int D, int ES>
struct DqDsCfg {
    static constexpr int NW = 4;
    static constexpr int NT = 64 * NW;
    static constexpr int BM = 32 * NW;                 // queries per workgroup
    static constexpr int BN = 128 / ES;                // keys per tile: 128 bytes of each dS row
    static constexpr int KW = D + (D == 64 ? 8 : 24);  // K rows, conflict-free transposing reads (as DqCfg)
    static constexpr int SW = (128 + 16) / ES;         // dS rows: 144 bytes (rows read at one column spread over the banks)
    using TS = typename std::conditional<ES == 4, float, T>::type;
    using KRows = DmaRowGroups<T, BN, D, KW, NW>;
    using SRows = DmaTile<TS, BM, BN, SW, NW>;
    static constexpr int KALLOC = BN * KW * (int)sizeof(T);
    static constexpr int BUF_BYTES = KALLOC + BM * SW * ES;
    static constexpr int NBUF = 2;
    static constexpr int OW = D + 8;
    static constexpr int STAGE_BYTES = NW * 32 * OW * (int)sizeof(T);
    static constexpr int SMEM_BYTES = NBUF * BUF_BYTES > STAGE_BYTES ? NBUF * BUF_BYTES : STAGE_BYTES;
    static_assert(2 * SMEM_BYTES <= 160 * 1024, "two workgroups per CU");
};

template <typename T, int D, bool CAUSAL, int ES>
__global__ __launch_bounds__(256, 2) void dq_ds_kernel(const BwdParams p, const int n_qtiles, const int fill) {
    using C = DqDsCfg<T, D, ES>;
    using TS = typename C::TS;
    static_assert(!Elem<T>::kF32, "16-bit inputs");
    static_assert(C::BM == DkdvCfg<T, D>::BK && C::BM == 128, "dS of the keys below a query tile's end is written");
    constexpr int BN = C::BN, KW = C::KW, SW = C::SW;
    __shared__ __attribute__((aligned(16))) char smem[C::SMEM_BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), l32 = lane & 31, hi = lane >> 5;
    const int2 tord = tile_order<64, CAUSAL>(n_qtiles);
    const int bh = tord.x;
    const int qt = n_qtiles - 1 - tord.y;  // longest causal rows first
    const int h = bh % p.H, b = bh / p.H;
    const int hk = h / p.group;
    const int q0 = qt * C::BM;
    const int qw0 = q0 + 32 * w;
    const int qi = qw0 + l32;

    f32x16 dq[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) dq[i] = f32x16{};

    // keys past the tile's last query have dS = 0 under the causal mask
    int kv_end = p.Sk;
    if (CAUSAL) kv_end = min(kv_end, q0 + C::BM);
    const int n_tiles = (kv_end + BN - 1) / BN;
    // tiles before n_plain need no masking for any row of the workgroup
    int n_plain = min(n_tiles, p.Sk / BN);
    if (CAUSAL) n_plain = min(n_plain, (q0 + 1) / BN);

    const T* kbase = (const T*)p.k + b * p.k_sb + hk * p.k_sh;
    const char* dsb = (const char*)p.dbias + (b * p.dbias_sb + h * p.dbias_sh) * ES;
    typename C::KRows krows;
    krows.init(p.k_ss, lane, w);
    typename C::SRows srows;
    srows.init(p.dbias_ss, lane, w);
    auto buf = [&](int s) -> char* { return smem + s * C::BUF_BYTES; };
    // tile j: K rows k0.., dS rows q0.. of keys k0.. (the descriptor's range
    // stops at the slice's readable end: rows past Sq land as zeros)
    auto issue = [&](int j, int s) FA_INLINE {
        const int k0 = j * BN;
        krows.load_untracked(kbase + (int64_t)k0 * p.k_ss, p.k_ss, p.Sk - k0, (const T*)buf(s));
        const int64_t toff = ((int64_t)q0 * p.dbias_ss + k0) * ES;
        const int64_t tlen = ((int64_t)(C::BM - 1) * p.dbias_ss + BN) * ES;
        const int bytes = (int)max((int64_t)0, min(tlen, (int64_t)p.ds_span - toff));
        srows.load_words(buffer_words(dsb + toff, bytes), (const TS*)(buf(s) + C::KALLOC));
    };
    auto sync_tiles = [&]() {
        wait_vmem();
        lds_barrier();
    };

    // ---- dQ^T += K^T dS^T for the tile in buffer s, 16 keys per step ----
    // lane (d, h) takes keys 16 ks + {4 h .. 4 h + 3, 8 + 4 h .. 8 + 4 h + 3},
    // the order of dq_kernel's products (the same sums, term by term): K^T by
    // two transposing reads of four K rows each, dS^T as two runs of four
    // elements of its query row
    const int trow = 4 * hi + ((lane & 15) >> 2);
    const int tcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    // keys of this lane's row at or past lim are zero (past Sk, or past the query)
    const int lim = CAUSAL ? min(p.Sk, qi + 1) : p.Sk;
    auto tile = [&](int j, int s, auto mask_tag) FA_INLINE {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int k0 = j * BN;
        if (MASK && CAUSAL && k0 > qw0 + 31) return;  // the wave's rows see none of these keys
        const T* Ks = (const T*)buf(s);
        const char* Ss = buf(s) + C::KALLOC + (32 * w + l32) * SW * ES;
#pragma unroll
        for (int ks = 0; ks < BN / 16; ++ks) {
            const int kl = 16 * ks + 4 * hi;  // tile-relative keys kl + 0..3 and kl + 8 + 0..3
            auto key = [&](int e) { return k0 + kl + (e < 4 ? e : 4 + e); };
            s16x8 bs;
            if constexpr (ES == 2) {
                bs = cat4(*reinterpret_cast<const s16x4*>(Ss + 2 * kl), *reinterpret_cast<const s16x4*>(Ss + 2 * kl + 16));
                if (MASK) {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (key(e) >= lim) bs[e] = 0;
                }
            } else {
                const f32x4 x0 = *reinterpret_cast<const f32x4*>(Ss + 4 * kl);
                const f32x4 x1 = *reinterpret_cast<const f32x4*>(Ss + 4 * kl + 32);
                float t8[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    t8[e] = x0[e];
                    t8[4 + e] = x1[e];
                }
                if (MASK) {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (key(e) >= lim) t8[e] = 0.f;
                }
                bs = pack8<T>(t8);
            }
#pragma unroll
            for (int i = 0; i < D / 32; ++i) {
                const T* kp = Ks + (16 * ks + trow) * KW + 32 * i + tcol;
                const s16x8 a = cat4(lds_read_tr16(kp), lds_read_tr16(kp + 8 * KW));
                dq[i] = Elem<T>::mfma(a, bs, dq[i]);
            }
        }
    };

    // two LDS buffers alternate: tile j is read from buffer j & 1 while tile
    // j + 1 is copied into the other one (last read in iteration j - 1, which
    // every wave finished before the opening barrier)
    int bcur = 0;
    if (n_tiles > 0) issue(0, 0);
    auto step = [&](int j, auto mask_tag) FA_INLINE {
        sync_tiles();
        if (j + 1 < n_tiles) issue(j + 1, bcur ^ 1);
        tile(j, bcur, mask_tag);
        bcur ^= 1;
    };
    for (int j = 0; j < n_plain; ++j) step(j, std::false_type{});
    for (int j = n_plain; j < n_tiles; ++j) step(j, std::true_type{});
    sync_tiles();  // every wave done with the tiles

    // ---- epilogue: stage dQ^T through LDS as rows, coalesced stores ----
    constexpr int OW = C::OW;
    T* Os = (T*)smem + w * 32 * OW;
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            s16x4 v4;
#pragma unroll
            for (int e = 0; e < 4; ++e) v4[e] = Elem<T>::pack1(dq[i][4 * g + e] * p.scale);
            *reinterpret_cast<s16x4*>(Os + l32 * OW + 32 * i + 8 * g + 4 * hi) = v4;
        }
    lds_barrier();
    constexpr int EPC = 16 / sizeof(T);
    constexpr int CPR = D / EPC;
    T* gbase = (T*)p.dq + b * p.dq_sb + h * p.dq_sh;
#pragma unroll
    for (int i = 0; i < 32 * CPR / 64; ++i) {
        const int cidx = lane + 64 * i;
        const int row = cidx / CPR, col = cidx % CPR;
        const int q = qw0 + row;
        if (q < p.Sq)
            *reinterpret_cast<uint4*>(gbase + (int64_t)q * p.dq_ss + col * EPC) =
                *reinterpret_cast<const uint4*>(Os + row * OW + col * EPC);
    }

    // ---- zeros of the gradient no kernel visits: keys from q0 + 128 on ----
    if (CAUSAL && fill) {
        const int kz = q0 + C::BM;
        const int nrow = min(C::BM, p.Sq - q0);
        if (kz < p.Sk) {
            const int cpr = (p.Sk - kz) * ES / 16;  // 16-byte chunks per row tail
            char* zb = (char*)p.dbias + (b * p.dbias_sb + h * p.dbias_sh + (int64_t)q0 * p.dbias_ss + kz) * ES;
            // non-temporal: nothing reads these lines back (C3 with a bias
            // gradient: 0.98 -> 0.94 ms for this pass)
            for (int r = w; r < nrow; r += C::NW)
                for (int c = lane; c < cpr; c += 64)
                    __builtin_nontemporal_store(u32x4{0u, 0u, 0u, 0u},
                                                reinterpret_cast<u32x4*>(zb + (int64_t)r * p.dbias_ss * ES + 16 * c));
        }
    }
}

// ---------------------------------------------------------------------------
// Whether the dK/dV stage runs dkdv8_kernel (16-bit inputs, no dropout, D >=
// 64): on grids of fewer workgroups than CUs, whose serial tile chain its two
// waves per SIMD halve, and with a bias at every grid size (two waves per SIMD
// where dkdv_kernel fits one), unless dkdv_kernel's per-element zero fill of
// the causal dBias is needed (rows not 16-byte aligned).
template <typename T, int D, bool CAUSAL, int DROPOUT, typename TB>
inline bool dkdv8_runs(const BwdParams& p) {
    if constexpr (!Elem<T>::kF32 && DROPOUT == 0 && D >= 64 && D <= 128) {
        constexpr bool BIAS = !std::is_void<TB>::value;
        const int64_t nb = (int64_t)((p.Sk + DkdvCfg<T, D>::BK - 1) / DkdvCfg<T, D>::BK) * p.Hkv * p.B;
        const bool fill1 = BIAS && CAUSAL && p.dbias != nullptr && p.dbias_zero_fill == 1;
        return nb > 0 && (nb < 256 || BIAS) && !fill1;
    }
    return false;
}

// Whether the dK/dV stage runs dkdv_pp_kernel (16-bit inputs, D = 128, no
// bias or dropout): one 8-wave workgroup per CU, so the grid must fill the CUs.
inline bool dkdv_pp_runs(const BwdParams& p) {
    const int64_t nb = (int64_t)((p.Sk + 255) / 256) * p.Hkv * p.B;
    return nb >= 256;
}

// Whether the dQ stage runs dq_pp_kernel (16-bit inputs, D = 128, no bias or
// dropout): one 8-wave workgroup of 256 queries per CU, so the grid must fill
// the CUs.
inline bool dq_pp_runs(const BwdParams& p) {
    const int64_t nb = (int64_t)((p.Sq + 255) / 256) * p.H * p.B;
    return nb >= 256;
}

// Whether the whole backward runs as the delta pre-pass plus bwd_small_kernel
// (16-bit inputs, D = 64 or 128, no bias or dropout): where dK/dV would run
// dkdv8_kernel on fewer workgroups than CUs and dQ the key-split dq_kernel,
// and either both kinds of workgroups fit the CUs at once or the mask makes
// their tile chains uneven (non-causal chains of one length on more workgroups
// than CUs gain nothing from sharing them and would pay the pre-pass).
template <typename T, int D, bool CAUSAL>
inline bool bwd_small_runs(const BwdParams& p) {
    if constexpr (!Elem<T>::kF32 && (D == 64 || D == 128) && 2 * DqCfg<T, D>::SMEM_BYTES <= 160 * 1024) {
        const int64_t nq = (int64_t)((p.Sq + DqCfg<T, D>::BM - 1) / DqCfg<T, D>::BM) * p.H * p.B;
        const int64_t nkv = (int64_t)((p.Sk + Dkdv8Cfg<T, D>::BK - 1) / Dkdv8Cfg<T, D>::BK) * p.Hkv * p.B;
        return dkdv8_runs<T, D, CAUSAL, 0, void>(p) && nq > 0 && nq < 256 && p.Sk > DqCfg<T, D>::BN &&
               (CAUSAL || nq + nkv <= 256);
    }
    return false;
}

template <typename T, int D, bool CAUSAL, int DROPOUT, typename TB>
hipError_t launch_bwd_t(const BwdParams& p0, int stage, hipStream_t s) {
    if constexpr (!Elem<T>::kF32 && DROPOUT == 0 && std::is_void<TB>::value && (D == 64 || D == 128)) {
        if (stage < 0 && bwd_small_runs<T, D, CAUSAL>(p0)) {
            hipError_t e = launch_bwd_t<T, D, CAUSAL, DROPOUT, TB>(p0, 0, s);  // delta rows
            if (e != hipSuccess) return e;
            BwdParams pr = p0;
            pr.dq_delta = 0;  // dQ reads the delta rows
            const int nk = (p0.Sk + Dkdv8Cfg<T, D>::BK - 1) / Dkdv8Cfg<T, D>::BK;
            const int nq = (p0.Sq + DqCfg<T, D>::BM - 1) / DqCfg<T, D>::BM;
            const int n_kv = nk * p0.Hkv * p0.B, n_q = nq * p0.H * p0.B;
            hipLaunchKernelGGL((bwd_small_kernel<T, D, CAUSAL>), dim3((unsigned)(n_kv + n_q)), dim3(512), 0, s, pr, nk,
                               n_kv, nq, n_q);
            return hipGetLastError();
        }
    }
    // stage 3: the workspace rows and dQ, for a dQ pass that recomputes dS.
    // 16-bit inputs do both in the dQ kernel (no delta pre-pass); fp32 runs
    // the pre-pass, then the dQ pass.  The whole backward without a dS pass
    // is stage 3, then dK/dV.
    const bool ds_pass = !std::is_void<TB>::value && !Elem<T>::kF32 && p0.dq_from_ds;
    if (stage == 3 || (stage < 0 && !ds_pass)) {
        hipError_t e;
        if constexpr (Elem<T>::kF32) {
            e = launch_bwd_t<T, D, CAUSAL, DROPOUT, TB>(p0, 0, s);
            if (e == hipSuccess) e = launch_bwd_t<T, D, CAUSAL, DROPOUT, TB>(p0, 2, s);
        } else {
            BwdParams pf = p0;
            pf.dq_delta = 1;
            e = launch_bwd_t<T, D, CAUSAL, DROPOUT, TB>(pf, 2, s);
        }
        if (e != hipSuccess || stage == 3) return e;
        return launch_bwd_t<T, D, CAUSAL, DROPOUT, TB>(p0, 1, s);
    }
    const BwdParams& p = p0;
    if (stage < 0 || stage == 0) {
        constexpr int EPC = 16 / sizeof(T);
        constexpr int RPB = 256 / (D / EPC);
        const int64_t nrows = (int64_t)p.B * p.sq_pad * p.H;
        const int64_t nb = (nrows + RPB - 1) / RPB;
        if (nb > 0) hipLaunchKernelGGL((delta_kernel<T, D>), dim3((unsigned)nb), dim3(256), 0, s, p);
    }
    if (stage < 0 || stage == 1) {
        using C = DkdvCfg<T, D>;
        const int nk = (p.Sk + C::BK - 1) / C::BK;
        const int64_t nb = (int64_t)nk * p.Hkv * p.B;
        bool done = false;
        if constexpr (!Elem<T>::kF32 && DROPOUT == 0 && std::is_void<TB>::value && D == 128) {
            if (dkdv_pp_runs(p)) {
                using CP = DkdvPPCfg<T, D>;
                const int nk2 = (p.Sk + CP::BK - 1) / CP::BK;
                const int64_t nb2 = (int64_t)nk2 * p.Hkv * p.B;
                hipLaunchKernelGGL((dkdv_pp_kernel<T, D, CAUSAL>), dim3((unsigned)nb2), dim3(CP::NT), 0, s, p, nk2);
                done = true;
            }
        }
        if constexpr (!Elem<T>::kF32 && DROPOUT == 0 && D >= 64 && D <= 128) {
            static_assert(Dkdv8Cfg<T, D>::BK == C::BK, "same key blocks");
            if (!done && dkdv8_runs<T, D, CAUSAL, DROPOUT, TB>(p)) {
                hipLaunchKernelGGL((dkdv8_kernel<T, D, CAUSAL, TB>), dim3((unsigned)nb), dim3(Dkdv8Cfg<T, D>::NT), 0, s, p,
                                   nk);
                done = true;
            }
        }
        if constexpr (D == 256) {
            // two launches of 128 dK / dV columns each (see dkdv_kernel)
            if (!done && nb > 0) {
                hipLaunchKernelGGL((dkdv_kernel<T, D, CAUSAL, DROPOUT, TB, 128, 0>), dim3((unsigned)nb), dim3(C::NT), 0, s,
                                   p, nk);
                hipLaunchKernelGGL((dkdv_kernel<T, D, CAUSAL, DROPOUT, TB, 128, 128>), dim3((unsigned)nb), dim3(C::NT), 0,
                                   s, p, nk);
            }
        } else {
            if (!done && nb > 0)
                hipLaunchKernelGGL((dkdv_kernel<T, D, CAUSAL, DROPOUT, TB>), dim3((unsigned)nb), dim3(C::NT), 0, s, p, nk);
        }
    }
    if (stage < 0 || stage == 2) {
        using C = DqCfg<T, D>;
        const int nq = (p.Sq + C::BM - 1) / C::BM;
        const int64_t nb = (int64_t)nq * p.H * p.B;
        bool done = false;
        // dS stored by the dK/dV pass: dQ = scale * dS K
        if constexpr (!Elem<T>::kF32 && !std::is_void<TB>::value) {
            if (p.dq_from_ds) {
                static_assert(DqDsCfg<T, D, 2>::BM == C::BM && DqDsCfg<T, D, 4>::BM == C::BM, "same query tiles");
                const int fill = p.dbias_zero_fill == 2;
                if (nb > 0) {
                    if (p.dbias_es == 4)
                        hipLaunchKernelGGL((dq_ds_kernel<T, D, CAUSAL, 4>), dim3((unsigned)nb), dim3(256), 0, s, p, nq, fill);
                    else
                        hipLaunchKernelGGL((dq_ds_kernel<T, D, CAUSAL, 2>), dim3((unsigned)nb), dim3(256), 0, s, p, nq, fill);
                }
                done = true;
            }
        }
        if constexpr (!Elem<T>::kF32 && DROPOUT == 0 && std::is_void<TB>::value && D == 128) {
            if (!done && dq_pp_runs(p)) {
                using CP = DqPPCfg<T, D>;
                const int64_t nb2 = (int64_t)((p.Sq + CP::BM - 1) / CP::BM) * p.H * p.B;
                hipLaunchKernelGGL((dq_pp_kernel<T, D, CAUSAL>), dim3((unsigned)nb2), dim3(CP::NT), 0, s, p);
                done = true;
            }
        }
        // grids of fewer workgroups than CUs split the key loop in two inside
        // the workgroup (as the forward does) where two splits' tiles fit the LDS
        if constexpr (2 * C::SMEM_BYTES <= 160 * 1024) {
            if (!done && nb > 0 && nb < 256 && p.Sk > C::BN) {
                hipLaunchKernelGGL((dq_kernel<T, D, CAUSAL, DROPOUT, TB, 2>), dim3((unsigned)nb), dim3(C::NT * 2), 0, s,
                                   p, nq);
                done = true;
            }
        }
        if (!done && nb > 0)
            hipLaunchKernelGGL((dq_kernel<T, D, CAUSAL, DROPOUT, TB, 1>), dim3((unsigned)nb), dim3(C::NT), 0, s, p, nq);
    }
    return hipGetLastError();
}

template <typename T, typename TB>
hipError_t launch_bwd_dispatch(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s) {
    // dropout mode: 0 none, 1 Philox mask regenerated, 2 the forward's keep bits read
    const int mode = !dropout ? 0 : (p.kb != nullptr ? 2 : 1);
#define FA_BWD_MODES(DD, CC)                                                \
    switch (mode) {                                                         \
        case 0: return launch_bwd_t<T, DD, CC, 0, TB>(p, stage, s);         \
        case 1: return launch_bwd_t<T, DD, CC, 1, TB>(p, stage, s);         \
        default: return launch_bwd_t<T, DD, CC, 2, TB>(p, stage, s);        \
    }
#define FA_BWD_CASE(DD)                                                     \
    if (D == DD) {                                                          \
        if (causal) FA_BWD_MODES(DD, true)                                  \
        FA_BWD_MODES(DD, false)                                             \
    }
    FA_BWD_CASE(32)
    FA_BWD_CASE(64)
    FA_BWD_CASE(128)
#undef FA_BWD_CASE
#undef FA_BWD_MODES
    return hipErrorInvalidValue;
}

// Head dim 256 (16-bit inputs, no bias): one workgroup per CU for dK/dV and
// dQ (translation units of their own, fa_bwd_d256_*.hip).
template <typename T>
hipError_t launch_bwd_d256(const BwdParams& p, bool causal, bool dropout, int stage, hipStream_t s) {
    static_assert(!Elem<T>::kF32, "16-bit inputs");
    const int mode = !dropout ? 0 : (p.kb != nullptr ? 2 : 1);
#define FA_BWD_MODES(CC)                                                    \
    switch (mode) {                                                         \
        case 0: return launch_bwd_t<T, 256, CC, 0, void>(p, stage, s);      \
        case 1: return launch_bwd_t<T, 256, CC, 1, void>(p, stage, s);      \
        default: return launch_bwd_t<T, 256, CC, 2, void>(p, stage, s);     \
    }
    if (causal) FA_BWD_MODES(true)
    FA_BWD_MODES(false)
#undef FA_BWD_MODES
}

}  // namespace fa
