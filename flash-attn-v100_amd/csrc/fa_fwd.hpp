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
//     copied global -> LDS directly (buffer_load ... lds) a full tile ahead.
//   * PV operands (V^T fragments) are read from the row-major V tile with
//     ds_read_b64_tr_b16, in the key order of the P accumulator layout.
//   * the loop is software-pipelined: S of the next tile is issued alongside
//     the softmax of the current one.
//   * exp2 with scale*log2(e) folded into one FMA; the running max is only
//     moved (and O rescaled) when it grows by more than 2^8, which is exact.
//   * causal: KV tiles past the last query are never loaded; tiles past a
//     wave's last query are skipped by that wave; only diagonal and tail tiles
//     run the masking variant of the tile step.
//   * fp32 inputs use v_mfma_f32_32x32x2_f32 with fp32 P.
//   * optional additive bias (BIAS): each lane reads 4 consecutive keys of its
//     query's bias row per load, issued a tile ahead; the scores become
//     t = S * scale + bias (one FMA) before the mask, and the softmax runs on
//     t with log2 e as its factor (reference forward_kernel.py:166-182).
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
    // V rows; 16-bit types read V^T fragments with ds_read_b64_tr_b16, whose
    // four rows per lane group fall in distinct banks at this stride
    static constexpr int VW = F32 ? D + 8 : D + (D == 64 ? 8 : 24);
    static constexpr int KTILE = BN * KW;
    static constexpr int VTILE = BN * VW;
    static constexpr int OW = D + (F32 ? 4 : 8);  // output staging row stride
    static constexpr int SMEM_ELEMS = 2 * (KTILE + VTILE);
    static_assert(NW * 32 * OW <= SMEM_ELEMS, "O staging must fit in the K/V buffers");
};

// TB: element type of the additive bias (T or float), void = no bias.
// KS: key split.  With KS > 1 the workgroup has KS groups of 4 waves on the
// same 128 queries; group sp walks key tiles sp, sp + KS, ... through its own
// double-buffered LDS tiles, and the partial (max, sum, O) of the groups are
// merged through LDS at the end (exactly: each part is rescaled to the common
// maximum).  Small grids use it: a workgroup's key loop is a serial chain of
// tile latencies, and KS groups walk it KS times shorter on the same CU.
// QG: query groups.  With QG = 2 (16-bit inputs and bias, no dropout, no key
// split) the workgroup has 2 groups of 4 waves on 256 queries, which share
// the K/V tiles, and each wave stages its bias rows through a private LDS
// region: 16-byte copies along the rows, where per-lane loads (one query row
// per lane) touch 32 rows per instruction.  The LDS of one such workgroup
// holds the K/V tiles and the 8 bias regions.
template <typename T, int D, bool CAUSAL, int DROPOUT, typename TB, int KS, int QG = 1>
__global__ __launch_bounds__(256 * KS * QG, KS == 1 && QG == 1 && D <= 128 ? 2 : 1) void fwd_kernel(const FwdParams p) {
    using C = FwdCfg<T, D>;
    constexpr bool BIAS = !std::is_void<TB>::value;
    using BT = typename std::conditional<BIAS, TB, T>::type;
    constexpr int BN = C::BN, NB = C::NB, KW = C::KW, VW = C::VW;
    constexpr bool BIAS_LDS = QG > 1;
    static_assert(QG == 1 || (QG == 2 && BIAS && !Elem<BT>::kF32 && !C::F32 && DROPOUT == 0 && KS == 1 && BN == 64),
                  "query groups: the staged 16-bit bias path");
    constexpr int BREG = 32 * 64;  // elements of a wave's bias region (32 rows of 64 keys)
    __shared__ __attribute__((aligned(16))) T smem[C::SMEM_ELEMS * KS + (BIAS_LDS ? 4 * QG * BREG : 0)];

    const int tid = threadIdx.x;
    // wave index as a scalar: loop bounds derived from it stay wave-uniform;
    // w: the wave's 32-query block, sp: its key split
    const int lane = tid & 63, wg = __builtin_amdgcn_readfirstlane(tid >> 6), l32 = lane & 31, hi = lane >> 5;
    // (compile-time 0 without a split: the compiler does not know the block
    // size); qg: the wave's query group
    const int w = KS == 1 && QG == 1 ? wg : wg & 3, sp = KS == 1 ? 0 : wg >> 2;
    const int qg = QG == 1 ? 0 : wg >> 2;

    // the divisor search for causal masking without a bias: the biased forward
    // keeps its code (measured 4 x 4096 x 32 heads with a full bias, where the
    // search keeps the group size, it was no faster)
    const int2 tord = tile_order<32 * (KS == 1 && QG == 1 && D <= 128 ? 2 : 1), CAUSAL && std::is_void<TB>::value>(p.n_qtiles);
    const int qt = p.n_qtiles - 1 - tord.y;  // longest causal rows first
    const int2 sbh = slice_bh(tord.x, p.H, p.B, !std::is_void<TB>::value && p.bias_sb == 0);
    const int h = sbh.y, b = sbh.x;
    const int hk = h / p.group;
    const int q0 = qt * C::BM * QG;  // the workgroup's first query
    const int qw0 = q0 + C::BM * qg + 32 * w;
    const int qi = qw0 + l32;

    const T* __restrict__ kbase = (const T*)p.k + b * p.k_sb + hk * p.k_sh;
    const T* __restrict__ vbase = (const T*)p.v + b * p.v_sb + hk * p.v_sh;

    int kv_end = p.Sk;
    if (CAUSAL) kv_end = min(kv_end, min(q0 + C::BM * QG, p.Sq));
    const int n_tiles = (kv_end + BN - 1) / BN;
    // tiles before n_plain need no masking for any wave of the workgroup
    int n_plain = min(n_tiles, p.Sk / BN);
    if (CAUSAL) n_plain = min(n_plain, (q0 + 1) / BN);
    // this split walks key tiles sp, sp + KS, ...: local tile j is key tile
    // j * KS + sp, and lc(n) counts the local tiles among the first n
    auto lc = [&](int n) { return n > sp ? (n - sp + KS - 1) / KS : 0; };
    auto key0 = [&](int j) { return (j * KS + sp) * BN; };

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
    // no wait here: the Q loads stay in flight while the first tile copies
    // are issued (the barrier before the first product waits for both)

    f32x16 o[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) o[i] = f32x16{};
    float m_run = -1e30f;  // running max in log2 units (scores * scale * log2 e)
    float l_run = 0.f;     // lane-partial row sum of exp2(t - m_run)
    float m_raw = -INFINITY;
    // score -> log2 units; with a bias the scores are scaled (and the bias
    // added) before the max, so the softmax factor is log2 e
    const float c = BIAS ? kLog2e : p.scale_log2;

    // ---- bias: 4-key groups {32 blk + 8 g + 4 hi + 0..3} of this lane's row ----
    // (rows past Sq read zeros; keys past Sk read zeros or the next row: masked)
    constexpr int NG = BIAS ? NB * 4 : 1;
    bias4_t<BT> bv[NG];
    const __amdgpu_buffer_rsrc_t brs =
        slice_buffer((const BT*)p.bias + b * p.bias_sb + h * p.bias_sh, BIAS ? p.bias_span : 0);
    const int bvoff = (qi * (int)p.bias_ss + 4 * hi) * (int)sizeof(BT);
    // staged bias (BIAS_LDS): copy chunk 64 t + lane of the wave's region is row
    // 8 t + lane / 8 at chunk position lane % 8, which holds key chunk
    // (lane % 8) ^ (lane / 8) of the row (keys 8 c .. 8 c + 7 of chunk c); rows
    // read 32 at one key chunk then fall in 8 distinct chunk positions.  Bias
    // rows are whole 16-byte chunks here (Sk % 8 == 0), so no copy straddles
    // the end of the slice.
    T* const bsm = smem + C::SMEM_ELEMS * KS + (BIAS_LDS ? wg * BREG : 0);
    const u32x4 bwords = buffer_words((const BT*)p.bias + b * p.bias_sb + h * p.bias_sh, BIAS_LDS ? p.bias_span : 0);
    const int bdoff = ((qw0 + (lane >> 3)) * (int)p.bias_ss + 8 * ((lane & 7) ^ (lane >> 3))) * (int)sizeof(BT);
    // a tile of plain iterations is always whole (MAYBE_TAIL = false)
    auto load_bias = [&](int k0, auto tail_tag) FA_INLINE {
        if constexpr (BIAS_LDS) {
            // the region was last read by this wave's add_bias of the previous tile
            const uint32_t l0 = lds_addr(bsm);
#pragma unroll
            for (int t = 0; t < 4; ++t)
                dma_load16_untracked(bwords, l0 + 1024 * t, bdoff + (8 * t * (int)p.bias_ss + k0) * (int)sizeof(BT));
        } else if constexpr (BIAS) {
            auto load_all = [&](auto full_tag) FA_INLINE {
#pragma unroll
                for (int g = 0; g < NG; ++g)
                    bv[g] = load_bias4<BT, decltype(full_tag)::value>(
                        brs, bvoff, (k0 + 32 * (g >> 2) + 8 * (g & 3)) * (int)sizeof(BT));
            };
            if (!decltype(tail_tag)::value || k0 + BN <= p.Sk)
                load_all(std::true_type{});
            else
                load_all(std::false_type{});
        }
    };
    // t = S * scale + bias
    auto add_bias = [&](f32x16 (&s)[NB]) FA_INLINE {
        if constexpr (BIAS_LDS) {
            wait_vmem();  // the wave's staged bias (and the tile copies issued before it)
            asm volatile("" ::: "memory");
#pragma unroll
            for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int c = 4 * blk + g;  // key chunk of registers 4 g .. 4 g + 3
                    const s16x4 v = *reinterpret_cast<const s16x4*>(bsm + l32 * 64 + 8 * (c ^ (l32 & 7)) + 4 * hi);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        s[blk][4 * g + e] = __builtin_fmaf(s[blk][4 * g + e], p.scale, bias_f32<BT>(v[e]));
                }
        } else if constexpr (BIAS) {
#pragma unroll
            for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    s[blk][r] = __builtin_fmaf(s[blk][r], p.scale, bias_f32<BT>(bv[4 * blk + (r >> 2)][r & 3]));
        }
    };

    // dropout: the mask drawn here (DROPOUT == 1), or read from the keep bits
    // written just before this kernel (DROPOUT == 2): the words of this lane's
    // query row for the 32-key blocks of a tile, loaded a tile ahead
    uint64_t row_ctr = 0;
    if (DROPOUT == 1) row_ctr = p.offset + ((uint64_t)(b * p.H + h) * (uint64_t)p.Sq + (uint64_t)qi) * (uint64_t)p.Sk;
    const uint32_t* kbrow = p.kb + (DROPOUT == 2 && qi < p.Sq ? ((int64_t)(b * p.H + h) * p.Sq + qi) * p.kb_w : 0);
    auto load_kb = [&](int k0, uint32_t (&wd)[NB]) FA_INLINE {
        if constexpr (DROPOUT == 2) {
#pragma unroll
            for (int blk = 0; blk < NB; ++blk)
                wd[blk] = qi < p.Sq && k0 + 32 * blk < p.Sk ? kbrow[(k0 >> 5) + blk] : 0u;
        }
    };

    T* Ks0 = smem + sp * C::SMEM_ELEMS;
    T* Vs0 = Ks0 + 2 * C::KTILE;
    // K and V tiles go global -> LDS directly and stay row-major.
    // Loads past the last key read as zeros (buffer range check), so the
    // pipeline below issues them unconditionally; such tiles are never used.
    const int wv = __builtin_amdgcn_readfirstlane(QG > 1 ? wg : w);
    DmaTile<T, BN, D, KW, C::NW * QG> kdma;
    kdma.init(p.k_ss, lane, wv);
    // 16-bit tiles: copies the compiler does not track, which it would
    // otherwise make the next LDS read wait for (sync_tiles waits for them)
    auto dma_k = [&](int j, int slot) {
        const int k0 = key0(j);
        if constexpr (C::F32)
            kdma.load(kbase + (int64_t)k0 * p.k_ss, p.k_ss, p.Sk - k0, Ks0 + slot * C::KTILE, lane);
        else
            kdma.load_untracked(kbase + (int64_t)k0 * p.k_ss, p.k_ss, p.Sk - k0, Ks0 + slot * C::KTILE, lane);
    };
    DmaTile<T, BN, D, VW, C::NW * QG> vst;
    vst.init(p.v_ss, lane, wv);
    auto load_v = [&](int j, int slot) {
        const int k0 = key0(j);
        if constexpr (C::F32)
            vst.load(vbase + (int64_t)k0 * p.v_ss, p.v_ss, p.Sk - k0, Vs0 + slot * C::VTILE, lane);
        else
            vst.load_untracked(vbase + (int64_t)k0 * p.v_ss, p.v_ss, p.Sk - k0, Vs0 + slot * C::VTILE, lane);
    };

    // ---- S^T = K Q^T for one key tile ----
    auto qk = [&](const T* Ks, f32x16 (&s)[NB]) {
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
    };
    // keys past Sk, and (causal) keys after the lane's query, to -inf
    auto mask = [&](f32x16 (&s)[NB], int k0) {
        const bool need = (k0 + BN > p.Sk) || (CAUSAL && k0 + BN - 1 > qw0);
        if (need) {
            // key k0 + 4 hi + o (o = 32 blk + 8 (r / 4) + r % 4) is masked when it is
            // >= Sk or (causal) > qi: one per-lane bound against constants
            const int lim = (CAUSAL ? min(p.Sk, qi + 1) : p.Sk) - k0 - 4 * hi;
#pragma unroll
            for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (32 * blk + 8 * (r >> 2) + (r & 3) >= lim) s[blk][r] = -INFINITY;
        }
    };
    // running max; O and l are rescaled (lazily: only when the max grows by
    // more than 2^8) before the tile's probabilities are added
    auto update_max = [&](const f32x16 (&s)[NB]) {
        float mx = -INFINITY;
#pragma unroll
        for (int blk = 0; blk < NB; ++blk)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[blk][r]);
        mx = pair_max(mx);
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
    };
    // P = exp2(S * scale * log2 e - m), row sums, dropout; 16-bit types pack P
    constexpr int NPK = C::F32 ? 1 : BN / 16;
    auto softmax = [&](f32x16 (&s)[NB], s16x8 (&pk)[NPK], int k0, const uint32_t (&wd)[NB]) {
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
                    const int kk = 8 * (r >> 2) + 4 * hi + (r & 3);
                    const bool keep = DROPOUT == 2
                                          ? ((wd[blk] >> kk) & 1u) != 0u
                                          : philox_keep(p.seed, row_ctr + (uint64_t)(k0 + 32 * blk + kk), p.keep_thresh);
                    if (!keep) s[blk][r] = 0.f;
                }
        }
        if constexpr (!C::F32) {
#pragma unroll
            for (int ks = 0; ks < BN / 16; ++ks) {
                float tmp[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) tmp[e] = s[ks >> 1][8 * (ks & 1) + e];
                pk[ks] = pack8<T>(tmp);
            }
        }
    };
    // ---- O^T += V^T P^T ----
    auto pv = [&](const T* Vs, const f32x16 (&s)[NB], const s16x8 (&pk)[NPK]) {
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
            for (int ks = 0; ks < BN / 16; ++ks)
#pragma unroll
                for (int i = 0; i < D / 32; ++i) {
                    // V^T fragment from the row-major tile: lane (d, h) takes keys
                    // 16 ks + {4h .. 4h+3, 8+4h .. 8+4h+3}, the keys of its P^T values
                    const T* vp = Vs + (16 * ks + 4 * hi + ((lane & 15) >> 2)) * VW + 32 * i + 16 * ((lane >> 4) & 1) +
                                  4 * (lane & 3);
                    const s16x8 a = cat4(lds_read_tr16(vp), lds_read_tr16(vp + 8 * VW));
                    o[i] = Elem<T>::mfma(a, pk[ks], o[i]);
                }
        }
    };

    // Software pipeline over key tiles.  Iteration j issues the MFMAs of
    // S(j+1) together with the softmax of S(j) (VALU), then P(j) V(j)
    // together with the max of S(j+1), so that the matrix pipe and the VALU
    // overlap inside one wave.
    //
    // LDS holds two K slots and two V slots.  Iteration j reads K(j+1) from
    // K slot (j+1)&1 and V(j) from V slot j&1, and copies K(j+2) into K slot
    // j&1 and V(j+1) into V slot (j+1)&1 -- both slots were last read in
    // iteration j-1, which every wave finished before the barrier that opens
    // iteration j.  Direct-to-LDS copies complete when the issuing wave's vmcnt drains, so
    // every barrier that publishes tiles is preceded by a wait for all of the
    // wave's outstanding loads (sync_tiles); the compiler only orders them
    // against the wave's own LDS reads.
    //
    // Waves whose queries all precede a key tile (causal) skip it; tiles
    // before n_plain need no mask for any wave of the workgroup.  Counts from
    // here on are of this split's local tiles.
    int n_w = n_tiles;
    if (CAUSAL) n_w = min(n_tiles, (qw0 + 31) / BN + 1);
    const int n_iter = (n_tiles + KS - 1) / KS;  // local tiles of split 0, the most of any split
    n_w = lc(n_w);
    n_plain = lc(n_plain);
    const int n_tl = lc(n_tiles);
    f32x16 sa[NB], sb[NB];
    s16x8 pk[NPK];
    uint32_t wa[NB], wb[NB];  // keep words of the current / next tile (DROPOUT == 2)

    auto sync_tiles = [&]() {
        wait_vmem();
        lds_barrier();
    };
    if (n_tl > 0) {
        dma_k(0, 0);
        dma_k(1, 1);
        load_v(0, 0);
    }
    sync_tiles();
    if (n_w > 0) {
        load_bias(key0(0), std::true_type{});
        load_kb(key0(0), wa);
        qk(Ks0, sa);
        add_bias(sa);
        if (n_plain == 0) mask(sa, key0(0));
        update_max(sa);
    }

    auto iter = [&](int j, f32x16 (&sc)[NB], f32x16 (&sn)[NB], const uint32_t (&wc)[NB], uint32_t (&wn)[NB],
                    auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        sync_tiles();
        dma_k(j + 2, j & 1);
        load_v(j + 1, (j + 1) & 1);
        const bool act = !MASK || j < n_w;
        const bool next = !MASK || j + 1 < n_w;
        if (act) {
            if (next) {
                load_bias(key0(j + 1), mask_tag);
                load_kb(key0(j + 1), wn);
                qk(Ks0 + ((j + 1) & 1) * C::KTILE, sn);
            }
            softmax(sc, pk, key0(j), wc);
        }
        if (act) pv(Vs0 + (j & 1) * C::VTILE, sc, pk);
        if (act && next) {
            add_bias(sn);
            if (MASK) mask(sn, key0(j + 1));
            update_max(sn);
        }
    };

    // plain iterations: S(j) and S(j+1) both unmasked (unrolled by two so
    // the score registers swap roles without copies)
    const int n_pipe = n_plain - 1;
    int j = 0;
    for (; j + 1 < n_pipe; j += 2) {
        iter(j, sa, sb, wa, wb, std::false_type{});
        iter(j + 1, sb, sa, wb, wa, std::false_type{});
    }
    if (j < n_pipe) {
        iter(j, sa, sb, wa, wb, std::false_type{});
        ++j;
#pragma unroll
        for (int blk = 0; blk < NB; ++blk) {
            sa[blk] = sb[blk];
            wa[blk] = wb[blk];
        }
    }
    for (; j + 1 < n_tl; j += 2) {
        iter(j, sa, sb, wa, wb, std::true_type{});
        iter(j + 1, sb, sa, wb, wa, std::true_type{});
    }
    if (j < n_tl) iter(j, sa, sb, wa, wb, std::true_type{});
    // splits with fewer tiles pass the barriers of the others' last iteration
    for (j = n_tl; j < n_iter; ++j) sync_tiles();

    sync_tiles();  // all waves done with the K/V buffers and no copy still in flight
    if constexpr (KS > 1) {
        // ---- merge the splits: parts of splits 1.. through LDS into split 0 ----
        constexpr int NO = (D / 32) * 16;  // O values per lane
        constexpr int NF = NO + 3;         // + running max, lane-partial sum, raw max
        static_assert((KS - 1) * 4 * NF * 64 * 4 <= (KS - 1) * C::SMEM_ELEMS * (int)sizeof(T),
                      "split parts fit the other splits' tile buffers");
        float* mg = reinterpret_cast<float*>(smem + C::SMEM_ELEMS);
        auto at = [&](int s2, int f) FA_INLINE { return mg + (((s2 - 1) * 4 + w) * NF + f) * 64 + lane; };
        if (sp > 0) {
#pragma unroll
            for (int i = 0; i < D / 32; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) *at(sp, 16 * i + r) = o[i][r];
            *at(sp, NO) = m_run;
            *at(sp, NO + 1) = l_run;
            *at(sp, NO + 2) = m_raw;
        }
        lds_barrier();
        if (sp == 0) {
            float mm = m_run;
#pragma unroll
            for (int s2 = 1; s2 < KS; ++s2) mm = fmaxf(mm, *at(s2, NO));
            const float a0 = fast_exp2(m_run - mm);
            l_run *= a0;
#pragma unroll
            for (int i = 0; i < D / 32; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[i][r] *= a0;
#pragma unroll
            for (int s2 = 1; s2 < KS; ++s2) {
                const float a = fast_exp2(*at(s2, NO) - mm);
                l_run = __builtin_fmaf(*at(s2, NO + 1), a, l_run);
                m_raw = fmaxf(m_raw, *at(s2, NO + 2));
#pragma unroll
                for (int i = 0; i < D / 32; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[i][r] = __builtin_fmaf(*at(s2, 16 * i + r), a, o[i][r]);
            }
            m_run = mm;
        }
    }

    // ---- epilogue: normalise, LSE, stage O^T through LDS, coalesced store ----
    // (split 0's waves; the others only pass the barriers)
    const float l_tot = pair_sum(l_run);
    const float inv = l_tot > 0.f ? (DROPOUT ? p.rp : 1.f) / l_tot : 0.f;
    if (sp == 0 && hi == 0 && qi < p.Sq) {
        const int64_t si = (int64_t)(b * p.H + h) * p.Sq + qi;
        p.lse[si] = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
        if (p.mx) p.mx[si] = BIAS ? m_raw : m_raw * p.scale;
    }
    constexpr int OW = C::OW;
    static_assert(C::NW * QG * 32 * OW <= C::SMEM_ELEMS, "O staging of every wave fits the K/V buffers");
    T* Os = smem + (QG > 1 ? wg : w) * 32 * OW;
    if (sp == 0) {
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
    }
    lds_barrier();
    constexpr int EPC = 16 / sizeof(T);
    constexpr int CPR = D / EPC;
    T* obase = (T*)p.o + b * p.o_sb + h * p.o_sh;
    if (sp == 0) {
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
}

// ---------------------------------------------------------------------------
// Ping-pong forward for 16-bit inputs without bias or dropout (the large-grid
// case).  One workgroup = 8 waves = 256 queries of one (batch, head); waves w
// and w + 4 run on the same SIMD (the hardware deals the waves of a workgroup
// to SIMDs 0, 2, 1, 3, 0, 2, 1, 3).  Every wave runs the same program,
//   for each key tile r:  M(r) | barrier | V(r) | barrier
//   M(r): S(r) = K(r) Q^T (if the wave needs key tile r), O^T += V(r-1)^T P(r-1)
//   V(r): mask (diagonal / tail tiles), running max, P(r) = exp2(...) packed
// but waves 4-7 pass one extra barrier first (and waves 0-3 one at the end),
// so the two waves of a SIMD run one phase apart: while one issues its matrix
// products, the other runs its softmax.  Every barrier is workgroup-wide.
// K and V tiles (global -> LDS, read by all 8 waves) rotate through four
// slots.  A ninth wave only copies them (issuing a tile's 36 copy
// instructions stalls the issuing wave for hundreds of cycles, which in a
// compute wave lengthens its phase): in round r it copies K(r+3) after the
// barrier that ends M(r) of waves 0-3 and V(r+2) after the one that ends
// their V(r), once its copies of round r-2 have landed, which that second
// barrier then publishes; a copy thus has two rounds to land, and a slot is
// only overwritten after both groups have read its previous tile.  Per query
// the arithmetic is that of fwd_kernel (same tile order, same lazy rescale per
// 32-query wave), so the outputs are bit-identical to it.
template <typename T, int D>
struct FwdPPCfg {
    static constexpr int NW = 8;                  // compute waves
    static constexpr int NT = 64 * (NW + 1);      // threads: the compute waves and the copy wave
    static constexpr int BM = 32 * NW;            // queries per workgroup
    static constexpr int BN = 64;                 // keys per tile
    static constexpr int NB = BN / 32;            // 32-key blocks per tile
    static constexpr int NSLOT = 4;               // K / V tile slots
    static constexpr int KW = D + 8;              // K row stride (elements)
    static constexpr int VW = D + (D == 64 ? 8 : 24);
    static constexpr int KTILE = BN * KW;
    static constexpr int VTILE = BN * VW;
    static constexpr int OW = D + 8;              // output staging row stride
    static constexpr int SMEM_ELEMS = NSLOT * (KTILE + VTILE);
    static_assert(NW * 32 * OW <= SMEM_ELEMS, "O staging must fit in the K/V buffers");
    static_assert(SMEM_ELEMS * 2 <= 160 * 1024, "LDS of one CU");
};

template <typename T, int D, bool CAUSAL, bool FIT>
__global__ __launch_bounds__(576, 1) void fwd_pp_kernel(const FwdParams p) {
    using C = FwdPPCfg<T, D>;
    static_assert(!Elem<T>::kF32, "16-bit inputs");
    constexpr int BN = C::BN, NB = C::NB, KW = C::KW, VW = C::VW, NSLOT = C::NSLOT;
    __shared__ __attribute__((aligned(16))) T smem[C::SMEM_ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), l32 = lane & 31, hi = lane >> 5;
    const int grp = w >> 2;
    // the two waves of a SIMD own adjacent 32-query blocks (similar causal work)
    const int blk = 2 * (w & 3) + grp;

    // FIT (the divisor search) only in the instantiation launched where it
    // changes the group size: with it this kernel's scalar registers moved and
    // it ran 2% slower at 4 x 4096 x 32 heads, causal, where it does not
    const int2 tord = tile_order<32, FIT>(p.n_qtiles);
    const int bh = tord.x;
    const int qt = p.n_qtiles - 1 - tord.y;  // longest causal rows first
    const int h = bh % p.H, b = bh / p.H;
    const int hk = h / p.group;
    const int q0 = qt * C::BM;
    const int qw0 = q0 + 32 * blk;
    const int qi = qw0 + l32;

    const T* __restrict__ kbase = (const T*)p.k + b * p.k_sb + hk * p.k_sh;
    const T* __restrict__ vbase = (const T*)p.v + b * p.v_sb + hk * p.v_sh;

    int kv_end = p.Sk;
    if (CAUSAL) kv_end = min(kv_end, min(q0 + C::BM, p.Sq));
    const int n_tiles = (kv_end + BN - 1) / BN;
    T* Ks0 = smem;
    T* Vs0 = smem + NSLOT * C::KTILE;

    if (w == C::NW) {
        // ---- the copy wave: the compute waves' barrier sequence, copies in between ----
        // round r (barriers 2r+1, 2r+2 after the prologue's): K(r+3) replaces
        // K(r-1) and V(r+2) replaces V(r-2), both last read in M(r-1), which
        // both groups have finished.  Tiles past Sk read nothing and land as
        // zeros.  At most 63 copy instructions are in flight (the vmcnt range).
        DmaTile<T, BN, D, KW, 1> kd;
        kd.init(p.k_ss, lane, 0);
        DmaTile<T, BN, D, VW, 1> vd;
        vd.init(p.v_ss, lane, 0);
        constexpr int NKI = decltype(kd)::NI, NVI = decltype(vd)::NI;
        static_assert(2 * NKI + NVI <= 63, "vmcnt range");
        // keys past the workgroup's last tile are never read: copies of tiles
        // from n_tiles on read nothing (empty range, zeros land) but are still
        // issued, so the vmcnt counts below stay exact
        const int k_lim = min(p.Sk, n_tiles * BN);
        lds_barrier();
        for (int r = 0; r <= n_tiles; ++r) {
            const int j = r + 3;
            barrier_no_fence();
            // round r-2's K(r+1), V(r) have landed (only round r-1's copies may
            // be in flight): the next barrier publishes them for M(r+1)
            wait_vmem_below<NKI + NVI>();
            kd.load_untracked(kbase + (int64_t)(j * BN) * p.k_ss, p.k_ss, k_lim - j * BN,
                              Ks0 + (j % NSLOT) * C::KTILE, lane);
            barrier_no_fence();
            wait_vmem_below<63 - NVI>();
            vd.load_untracked(vbase + (int64_t)((j - 1) * BN) * p.v_ss, p.v_ss, k_lim - (j - 1) * BN,
                              Vs0 + ((j - 1) % NSLOT) * C::VTILE, lane);
        }
        barrier_no_fence();  // the one waves 0-3 pass after their last round
        wait_vmem();         // every copy has landed before the slots hold O
        lds_barrier();
        lds_barrier();
        return;
    }

    // key tiles this wave uses, and how many of them need no mask
    int n_w = qw0 < p.Sq ? n_tiles : 0;
    if (CAUSAL) n_w = min(n_w, (qw0 + 31) / BN + 1);
    int n_um = min(n_w, p.Sk / BN);
    if (CAUSAL) n_um = min(n_um, (qw0 + 1) / BN);

    // ---- Q into registers (MFMA B operand): d = 16 i + 8 hi .. +7 ----
    constexpr int QR = D / 16;
    uint4 qreg[QR];
    {
        const T* qrow = (const T*)p.q + b * p.q_sb + (int64_t)qi * p.q_ss + h * p.q_sh;
#pragma unroll
        for (int i = 0; i < QR; ++i)
            qreg[i] = qi < p.Sq ? *reinterpret_cast<const uint4*>(qrow + 16 * i + 8 * hi) : make_uint4(0u, 0u, 0u, 0u);
    }

    f32x16 o[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) o[i] = f32x16{};
    float m_run = -1e30f;  // running max in log2 units
    float l_run = 0.f;     // lane-partial row sum
    float m_raw = -INFINITY;
    const float c = p.scale_log2;

    // prologue copies: the 8 compute waves (in the loop: the copy wave)
    DmaTile<T, BN, D, KW, C::NW> kdma;
    kdma.init(p.k_ss, lane, w);
    DmaTile<T, BN, D, VW, C::NW> vdma;
    vdma.init(p.v_ss, lane, w);
    auto dma_k = [&](int j) FA_INLINE {
        if (j < n_tiles)
            kdma.load(kbase + (int64_t)(j * BN) * p.k_ss, p.k_ss, p.Sk - j * BN, Ks0 + (j % NSLOT) * C::KTILE, lane);
    };
    auto dma_v = [&](int j) FA_INLINE {
        if (j < n_tiles)
            vdma.load(vbase + (int64_t)(j * BN) * p.v_ss, p.v_ss, p.Sk - j * BN, Vs0 + (j % NSLOT) * C::VTILE, lane);
    };
    f32x16 s[NB];       // scores of tile r between its M and V phases
    s16x8 pk[BN / 16];   // P of tile r between its V phase and the M phase of tile r+1

    // ---- M phase of tile r: S(r) = K(r) Q^T, O^T += V(r-1)^T P(r-1) ----
    // Step t issues the t-th S product and the t-th PV product; the LDS
    // operands of step t + MP are read during step t (MP steps ahead), so no
    // product waits out an LDS latency.
    const int trow = 4 * hi + ((lane & 15) >> 2);
    const int tcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    constexpr int NQK = NB * QR;               // S MFMAs per tile
    constexpr int NPV = (BN / 16) * (D / 32);  // PV MFMAs per tile
    static_assert(NQK == NPV, "one S and one PV product per step");
    constexpr int NSTEP = NQK;
    constexpr int MP = 2;  // measured against 1, 3, 4, 5 (3: 1-2% slower, 1: 7%)
    auto kfrag = [&](const T* Ks, int t) FA_INLINE {
        const int bk = t / QR, kk = t % QR;
        return *reinterpret_cast<const s16x8*>(Ks + (32 * bk + l32) * KW + 16 * kk + 8 * hi);
    };
    auto vfrag = [&](const T* Vs, int t) FA_INLINE {
        const int ks = t / (D / 32), i = t % (D / 32);
        const T* vp = Vs + (16 * ks + trow) * VW + 32 * i + tcol;
        return cat4(lds_read_tr16(vp), lds_read_tr16(vp + 8 * VW));
    };
    auto qk_mfma = [&](const s16x8& a, int t) FA_INLINE {
        const int bk = t / QR, kk = t % QR;
        s[bk] = Elem<T>::mfma(a, __builtin_bit_cast(s16x8, qreg[kk]), kk == 0 ? f32x16{} : s[bk]);
    };
    auto pv_mfma = [&](const s16x8& a, int t) FA_INLINE {
        const int ks = t / (D / 32), i = t % (D / 32);
        o[i] = Elem<T>::mfma(a, pk[ks], o[i]);
    };
    // QK: S(r) only (the first tile); PV: O += V(r-1) P(r-1) only (the tile after a wave's last)
    auto mphase = [&](int r, auto qk_tag, auto pv_tag) FA_INLINE {
        constexpr bool QK = decltype(qk_tag)::value, PV = decltype(pv_tag)::value;
        const T* Ks = Ks0 + (r % NSLOT) * C::KTILE;
        const T* Vs = Vs0 + ((r + NSLOT - 1) % NSLOT) * C::VTILE;
        s16x8 kf[NSTEP], vf[NSTEP];
#pragma unroll
        for (int t = 0; t < MP; ++t) {
            if (QK) kf[t] = kfrag(Ks, t);
            if (PV) vf[t] = vfrag(Vs, t);
        }
#pragma unroll
        for (int t = 0; t < NSTEP; ++t) {
            if (t + MP < NSTEP) {
                if (QK) kf[t + MP] = kfrag(Ks, t + MP);
                if (PV) vf[t + MP] = vfrag(Vs, t + MP);
            }
            if (QK) qk_mfma(kf[t], t);
            if (PV) pv_mfma(vf[t], t);
        }
        // the same order for the scheduler: reads of MP steps, then per step
        // its products followed by the reads of step t + MP
        constexpr int RD = (QK ? 1 : 0) + (PV ? 2 : 0);
        constexpr int MF = (QK ? 1 : 0) + (PV ? 1 : 0);
#pragma unroll
        for (int t = 0; t < MP; ++t) __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);
#pragma unroll
        for (int t = 0; t < NSTEP; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, MF, 0);
            if (t + MP < NSTEP) __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);
        }
    };

    // ---- V phase of tile r: mask, running max (lazy rescale), P(r) ----
    const int lim0 = (CAUSAL ? min(p.Sk, qi + 1) : p.Sk) - 4 * hi;
    auto vphase = [&](int r) FA_INLINE {
        if (r >= n_um) {
            // key r BN + 4 hi + o (o = 32 bk + 8 (e / 4) + e % 4) is masked when it
            // is >= Sk or (causal) > qi: one per-lane bound against constants
            const int lim = lim0 - r * BN;
#pragma unroll
            for (int bk = 0; bk < NB; ++bk)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    if (32 * bk + 8 * (e >> 2) + (e & 3) >= lim) s[bk][e] = -INFINITY;
        }
        float mx = -INFINITY;
#pragma unroll
        for (int bk = 0; bk < NB; ++bk)
#pragma unroll
            for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[bk][e]);
        mx = pair_max(mx);
        m_raw = fmaxf(m_raw, mx);
        const float m_new = fmaxf(m_run, mx * c);
        if (__ballot(m_new > m_run + 8.0f) != 0ull) {
            const float alpha = fast_exp2(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < D / 32; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
            m_run = m_new;
        }
        float psum = 0.f;
#pragma unroll
        for (int bk = 0; bk < NB; ++bk)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float pv = fast_exp2(__builtin_fmaf(s[bk][e], c, -m_run));
                psum += pv;
                s[bk][e] = pv;
            }
        l_run += psum;
#pragma unroll
        for (int ks = 0; ks < BN / 16; ++ks) {
            float tmp[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) tmp[e] = s[ks >> 1][8 * (ks & 1) + e];
            pk[ks] = pack8<T>(tmp);
        }
    };

    auto sched_fence = [&]() FA_INLINE { __builtin_amdgcn_sched_barrier(0); };
    // one round: M phase, barrier, V phase, barrier (the copy wave issues the
    // tile copies between them; no release fence: the copies are ordered by
    // the copy wave's vmcnt waits, and every LDS read of M(r) has completed,
    // its products consumed it)
    auto round = [&](int r, auto qk_tag, auto pv_tag, auto v_tag) FA_INLINE {
        sched_fence();
        if constexpr (decltype(qk_tag)::value || decltype(pv_tag)::value) mphase(r, qk_tag, pv_tag);
        sched_fence();
        barrier_no_fence();
        sched_fence();
        if constexpr (decltype(v_tag)::value) vphase(r);
        sched_fence();
        barrier_no_fence();
    };
    using TT = std::true_type;
    using FF = std::false_type;

    // prologue: the tiles the first three M phases read
    dma_k(0);
    dma_k(1);
    dma_k(2);
    dma_v(0);
    dma_v(1);
    wait_vmem();
    lds_barrier();
    if (grp == 1) barrier_no_fence();  // waves 4-7 run one phase behind
    // rounds 0 .. n_tiles: S(0) alone; S(r) with P(r-1) V(r-1) while the wave
    // needs tile r; P V of its last tile; then only the copies
    int r = 0;
    if (n_w > 0) {
        round(0, TT{}, FF{}, TT{});
        for (r = 1; r < n_w; ++r) round(r, TT{}, TT{}, TT{});
        round(r, FF{}, TT{}, FF{});
        ++r;
    }
    for (; r <= n_tiles; ++r) round(r, FF{}, FF{}, FF{});
    if (grp == 0) barrier_no_fence();
    sched_fence();

    // ---- epilogue: normalise, LSE, stage O^T through LDS, coalesced store ----
    const float l_tot = pair_sum(l_run);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (hi == 0 && qi < p.Sq) {
        const int64_t si = (int64_t)(b * p.H + h) * p.Sq + qi;
        p.lse[si] = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
        if (p.mx) p.mx[si] = m_raw * p.scale;
    }
    lds_barrier();   // every wave is done with the K / V slots, every copy landed
    constexpr int OW = C::OW;
    T* Os = smem + w * 32 * OW;
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * i + 8 * g + 4 * hi;
            s16x4 v4;
#pragma unroll
            for (int e = 0; e < 4; ++e) v4[e] = Elem<T>::pack1(o[i][4 * g + e] * inv);
            *reinterpret_cast<s16x4*>(Os + l32 * OW + d) = v4;
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

// When the ping-pong kernel runs (measured, D = 128, bf16, interleaved A/B
// against fwd_kernel): its 256-query workgroups must fill the chip at least
// once, and with causal masking it needs long rows and a grid that fills the
// chip twice (it runs one workgroup per CU, so the causal diagonal, where the
// waves of the lower query blocks have no work, and each workgroup's first
// tile copies are not hidden by a second workgroup).  Causal: (1, 4096, 32)
// -12%, (1, 8192, 16) -14%, (2, 3072, 32) -6%; (1, 4096, 16) and (1, 8192, 8)
// (256 workgroups) +3%, (4, 2048, 32) and (2, 2048, 64) equal, (8, 1024, 32)
// +3%.
// The causal fwd_pp_kernel with FIT (D = 128), instantiated in a translation
// unit of its own (fa_fwd_fit.hip), so that the units of the plain kernels
// compile the same code as without it (their prologues' instruction order
// has moved with unrelated changes, and the forward's speed with it)
template <typename T>
hipError_t launch_fwd_pp_fit(const FwdParams& q, int64_t nblocks, hipStream_t s);

inline bool fwd_pp_wanted(const FwdParams& p, bool causal) {
    const int64_t n = (int64_t)((p.Sq + 255) / 256) * p.H * p.B;
    return n >= 256 && (!causal || (p.Sq >= 3072 && n >= 512));
}

template <typename T, int D, bool CAUSAL, int DROPOUT, typename TB>
hipError_t launch_fwd_t(const FwdParams& p, hipStream_t s) {
    if constexpr (!Elem<T>::kF32 && DROPOUT == 0 && std::is_void<TB>::value && D == 128) {
        if (fwd_pp_wanted(p, CAUSAL)) {
            using CP = FwdPPCfg<T, D>;
            FwdParams q = p;
            q.n_qtiles = (p.Sq + CP::BM - 1) / CP::BM;
            const int64_t nblocks = (int64_t)q.n_qtiles * p.H * p.B;
            // causal rows differ in length, so a small last slice group runs
            // its long rows alone: (2, 3072, 32) 173.0 -> 155.7 us with FIT
            if constexpr (CAUSAL) {
                if (host_group_uneven(32, q.n_qtiles, (int)nblocks)) return launch_fwd_pp_fit<T>(q, nblocks, s);
            }
            hipLaunchKernelGGL((fwd_pp_kernel<T, D, CAUSAL, false>), dim3((unsigned)nblocks), dim3(CP::NT), 0, s, q);
            return hipGetLastError();
        }
    }
    using C = FwdCfg<T, D>;
    // a 16-bit bias without dropout: 256-query workgroups that stage the bias
    // through LDS, where the grid still fills the CUs and bias rows are whole
    // 16-byte chunks
    if constexpr (!Elem<T>::kF32 && DROPOUT == 0 && !std::is_void<TB>::value) {
        if constexpr (!Elem<TB>::kF32) {
            FwdParams q = p;
            q.n_qtiles = (p.Sq + 2 * C::BM - 1) / (2 * C::BM);
            const int64_t nb2 = (int64_t)q.n_qtiles * p.H * p.B;
            if (nb2 >= 256 && p.Sk % 8 == 0) {
                hipLaunchKernelGGL((fwd_kernel<T, D, CAUSAL, 0, TB, 1, 2>), dim3((unsigned)nb2), dim3(C::NT * 2), 0, s, q);
                return hipGetLastError();
            }
        }
    }
    FwdParams q = p;
    q.n_qtiles = (p.Sq + C::BM - 1) / C::BM;
    const int64_t nblocks = (int64_t)q.n_qtiles * p.H * p.B;
    if (nblocks <= 0) return hipSuccess;
    // grids that leave CUs idle split the key loop inside the workgroup: into
    // 4 where four splits fit 128 registers a lane without spilling (16-bit,
    // D = 32, no dropout, no bias), else into 2
    constexpr int KS_SMALL = (!Elem<T>::kF32 && D == 32 && DROPOUT == 0 && std::is_void<TB>::value) ? 4 : 2;
    const int n_cu = 256;
    // (D = 256: one workgroup's tiles take most of the LDS, no split)
    if constexpr (D <= 128) {
        if (nblocks < n_cu && p.Sk > C::BN) {
            hipLaunchKernelGGL((fwd_kernel<T, D, CAUSAL, DROPOUT, TB, KS_SMALL>), dim3((unsigned)nblocks),
                               dim3(C::NT * KS_SMALL), 0, s, q);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((fwd_kernel<T, D, CAUSAL, DROPOUT, TB, 1>), dim3((unsigned)nblocks), dim3(C::NT), 0, s, q);
    return hipGetLastError();
}

template <typename T, typename TB>
hipError_t launch_fwd_dispatch(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s) {
    // dropout mode: 0 none, 1 Philox mask, 2 Philox mask also written as keep bits
    const int mode = !dropout ? 0 : (p.kb != nullptr ? 2 : 1);
#define FA_FWD_MODES(DD, CC)                                                \
    switch (mode) {                                                         \
        case 0: return launch_fwd_t<T, DD, CC, 0, TB>(p, s);                \
        case 1: return launch_fwd_t<T, DD, CC, 1, TB>(p, s);                \
        default: return launch_fwd_t<T, DD, CC, 2, TB>(p, s);               \
    }
#define FA_FWD_CASE(DD)                                                     \
    if (D == DD) {                                                          \
        if (causal) FA_FWD_MODES(DD, true)                                  \
        FA_FWD_MODES(DD, false)                                             \
    }
    FA_FWD_CASE(32)
    FA_FWD_CASE(64)
    FA_FWD_CASE(128)
#undef FA_FWD_CASE
#undef FA_FWD_MODES
    return hipErrorInvalidValue;
}

// Head dim 256 (16-bit inputs, no bias): one workgroup of 4 waves per CU, the
// Q rows and O accumulators of a wave in 192 registers (translation units of
// their own, fa_fwd_d256_*.hip).
template <typename T>
hipError_t launch_fwd_d256(const FwdParams& p, bool causal, bool dropout, hipStream_t s) {
    static_assert(!Elem<T>::kF32, "16-bit inputs");
    const int mode = !dropout ? 0 : (p.kb != nullptr ? 2 : 1);
#define FA_FWD_MODES(CC)                                                    \
    switch (mode) {                                                         \
        case 0: return launch_fwd_t<T, 256, CC, 0, void>(p, s);             \
        case 1: return launch_fwd_t<T, 256, CC, 1, void>(p, s);             \
        default: return launch_fwd_t<T, 256, CC, 2, void>(p, s);            \
    }
    if (causal) FA_FWD_MODES(true)
    FA_FWD_MODES(false)
#undef FA_FWD_MODES
}

}  // namespace fa
