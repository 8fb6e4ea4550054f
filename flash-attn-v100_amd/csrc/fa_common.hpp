// Device-side building blocks shared by the gfx950 attention kernels.
//
// Wave64 MFMA operand layouts used throughout (checked on gfx950):
//   v_mfma_f32_32x32x16_{bf16,f16}: lane l holds A[l%32][8*(l/32) + e] and
//     B[8*(l/32) + e][l%32] for e = 0..7; accumulator r (0..15) of lane l is
//     C[8*(r/4) + 4*(l/32) + r%4][l%32].
//   v_mfma_f32_32x32x2_f32: lane l holds A[l%32][l/32], B[l/32][l%32]; same C.
//   ds_read_b64_tr_b16: inside each 16-lane group, output lane i element e is
//     element i%4 of the 8 bytes addressed by lane 4*e + i/4 of the group.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

// Device helpers and kernel-local lambdas are always inlined: an out-of-line
// call would keep tile descriptors and MFMA accumulators in scratch memory
// (and turn wave-uniform buffer descriptors into per-lane ones).
#define FA_INLINE __attribute__((always_inline))

namespace fa {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------
// element traits
template <typename T> struct Elem;
template <> struct Elem<bf16> {
    static constexpr bool kF32 = false;
    using Vec8 = bf16x8;
    __device__ FA_INLINE static inline f32x16 mfma(const s16x8& a, const s16x8& b, const f32x16& c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
    __device__ FA_INLINE static inline short pack1(float x) { return __builtin_bit_cast(short, (bf16)x); }
    __device__ FA_INLINE static inline float unpack1(short x) { return (float)__builtin_bit_cast(bf16, x); }
};
template <> struct Elem<f16> {
    static constexpr bool kF32 = false;
    using Vec8 = f16x8;
    __device__ FA_INLINE static inline f32x16 mfma(const s16x8& a, const s16x8& b, const f32x16& c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
    __device__ FA_INLINE static inline short pack1(float x) { return __builtin_bit_cast(short, (f16)x); }
    __device__ FA_INLINE static inline float unpack1(short x) { return (float)__builtin_bit_cast(f16, x); }
};
template <> struct Elem<float> {
    static constexpr bool kF32 = true;
};

__device__ FA_INLINE inline f32x16 mfma_f32(float a, float b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// 8 x 16-bit elements <-> 8 floats
template <typename T>
__device__ FA_INLINE inline s16x8 pack8(const float* x) {
    s16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = Elem<T>::pack1(x[e]);
    return r;
}

// Reductions over the lane pair (l, l^32) with one v_permlane32_swap (no LDS
// round trip).  Swapping x with itself leaves x[l%32] in one result and
// x[l%32 + 32] in the other for every lane, so max / sum of the two results is
// the pair reduction in all 64 lanes without a per-half select.  The second
// result passes through a register move the compiler cannot see through: it
// otherwise folds max(r0, r1) and r0 + r1 as if both results were x.
__device__ FA_INLINE inline void pair_swap(float x, float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x),
                                                    false, false);
    unsigned hidden;
    asm volatile("v_mov_b32 %0, %1" : "=v"(hidden) : "v"(r[1]));
    a = __builtin_bit_cast(float, (unsigned)r[0]);
    b = __builtin_bit_cast(float, hidden);
}
__device__ FA_INLINE inline float pair_max(float x) {
    float a, b;
    pair_swap(x, a, b);
    return fmaxf(a, b);
}
__device__ FA_INLINE inline float pair_sum(float x) {
    float a, b;
    pair_swap(x, a, b);
    return a + b;
}

// x of lane `lane ^ S` (S = 1, 2, 4, 8, 16): DPP moves within rows of 16
// lanes (quad permutes for 1 and 2; row shifts up / down, one per side, for
// 4 and 8), v_permlane16_swap between the rows of each 32-lane half for 16
template <int S>
__device__ FA_INLINE inline uint32_t xor_lane(uint32_t x, int lane) {
    const int v = (int)x;
    if constexpr (S == 1) {
        return (uint32_t)__builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (S == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (S == 4 || S == 8) {
        const int up = __builtin_amdgcn_update_dpp(v, v, 0x100 + S, 0xF, 0xF, false);  // row_shl: lane + S
        const int dn = __builtin_amdgcn_update_dpp(v, v, 0x110 + S, 0xF, 0xF, false);  // row_shr: lane - S
        return (uint32_t)((lane & S) ? dn : up);
    } else {
        static_assert(S == 16, "lane distance");
        const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        // r[0] holds lane - 16 in the odd rows, r[1] lane + 16 in the even rows
        return (lane & 16) ? (uint32_t)r[0] : (uint32_t)r[1];
    }
}

// 32 x 32 bit-matrix transpose within each 32-lane half: lane L holds row
// word w (bit j = element (L, j)); afterwards lane j holds column word j (bit
// L = element (L, j)).  Stage S swaps the off-diagonal S x S blocks between
// lanes L and L ^ S.
template <int S, uint32_t M>
__device__ FA_INLINE inline uint32_t transpose_stage(uint32_t w, int lane) {
    const uint32_t o = xor_lane<S>(w, lane);
    return (lane & S) ? ((w & ~M) | ((o >> S) & M)) : ((w & M) | ((o & M) << S));
}
__device__ FA_INLINE inline uint32_t transpose32(uint32_t w, int lane) {
    w = transpose_stage<16, 0x0000FFFFu>(w, lane);
    w = transpose_stage<8, 0x00FF00FFu>(w, lane);
    w = transpose_stage<4, 0x0F0F0F0Fu>(w, lane);
    w = transpose_stage<2, 0x33333333u>(w, lane);
    return transpose_stage<1, 0x55555555u>(w, lane);
}

__device__ FA_INLINE inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------
// additive bias (element type T, key stride 1)
// Four consecutive keys of one bias row in raw form (one 8- or 16-byte load).
template <typename T>
using bias4_t = typename std::conditional<Elem<T>::kF32, f32x4, s16x4>::type;

// A (batch, head) slice of the bias (or of its gradient) is addressed through
// a buffer resource whose range is the slice's byte span: reads past it
// return 0 and writes past it are dropped, so per-lane offsets need no bounds
// checks and stay 32-bit (the host bounds every offset below 2^31).
template <typename T>
__device__ FA_INLINE inline __amdgpu_buffer_rsrc_t slice_buffer(const T* base, int span_bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, span_bytes, 0x00020000);
}

// Four consecutive keys at byte offset voff + soff.  full: one 8- or 16-byte
// load.  A load that straddles the end of the range reads as all zeros, so a
// tile that holds the last key of a row (the last row of a slice may end
// inside a group of four) loads key by key instead.
template <typename T, bool FULL>
__device__ FA_INLINE inline bias4_t<T> load_bias4(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
    if constexpr (FULL) {
        if constexpr (Elem<T>::kF32)
            return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0));
        else
            return __builtin_bit_cast(s16x4, __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, 0));
    } else {
        bias4_t<T> v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if constexpr (Elem<T>::kF32)
                v[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff + 4 * e, 0));
            else
                v[e] = (short)__builtin_amdgcn_raw_buffer_load_b16(rs, voff, soff + 2 * e, 0);
        }
        return v;
    }
}

// raw bias element -> float
template <typename T>
__device__ FA_INLINE inline float bias_f32(float x) { return x; }
template <typename T>
__device__ FA_INLINE inline float bias_f32(short x) { return Elem<T>::unpack1(x); }

// one raw bias element (16-bit types as short)
template <typename T>
using bias1_t = typename std::conditional<Elem<T>::kF32, float, short>::type;
template <typename T>
__device__ FA_INLINE inline bias1_t<T> load_bias1(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
    if constexpr (Elem<T>::kF32)
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, 0));
    else
        return (short)__builtin_amdgcn_raw_buffer_load_b16(rs, voff, soff, 0);
}

// one gradient element at byte offset voff + soff (dropped past the range),
// rounded to DT (0 fp16, 1 bf16, 2 fp32)
template <int DT>
__device__ FA_INLINE inline void store_grad(__amdgpu_buffer_rsrc_t rs, float x, int voff, int soff) {
    if constexpr (DT == 2)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, x), rs, voff, soff, 0);
    else if constexpr (DT == 1)
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (bf16)x), rs, voff, soff, 0);
    else
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (f16)x), rs, voff, soff, 0);
}
// f(std::integral_constant<int, DT>) for the wave-uniform runtime dtype code,
// so that a block of stores branches once
template <typename F>
__device__ FA_INLINE inline void with_grad_dtype(int dtype, F&& f) {
    if (dtype == 2)
        f(std::integral_constant<int, 2>{});
    else if (dtype == 1)
        f(std::integral_constant<int, 1>{});
    else
        f(std::integral_constant<int, 0>{});
}
// a lane offset that lands every access of the lane out of range (offsets
// past it stay below 2^32, so they cannot wrap back into the range)
constexpr int kOffNowhere = (int)0x80000000u;

// Workgroup barrier that orders LDS only.  __syncthreads() also fences global
// memory, which on gfx9 (one counter for vector loads and stores) makes every
// barrier wait for the in-flight prefetch of the next tile; the kernels never
// communicate through global memory, so an LDS-scoped fence is sufficient.
__device__ FA_INLINE inline void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Workgroup barrier without a memory fence, for loops that order their LDS
// traffic explicitly: a release fence would make the compiler wait for every
// direct-to-LDS copy still in flight (vmcnt(0)), including copies issued just
// before the barrier for a later tile.  The empty asm statements keep the
// compiler from moving memory accesses across the barrier.
__device__ FA_INLINE inline void barrier_no_fence() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// LDS access
typedef __attribute__((address_space(3))) void lds_void;

// p must point into __shared__ memory (8-byte aligned); the cast is an
// address-space cast, not an integer reinterpretation.
__device__ FA_INLINE inline s16x4 lds_read_tr16(const void* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}

__device__ FA_INLINE inline s16x8 cat4(const s16x4& a, const s16x4& b) {
    s16x8 r;
    r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
    r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
    return r;
}

// ---------------------------------------------------------------------------
// Philox4x32-10 (Salmon et al., SC'11) with Triton's tl.rand conventions:
// key = (lo32 seed, hi32 seed), counter = (lo32 c, hi32 c, 0, 0); word 0 is
// bit-cast to int32, folded x < 0 ? -x - 1 : x, and scaled by 4.6566127342e-10.
__device__ FA_INLINE inline uint32_t philox_word0(uint64_t seed, uint64_t ctr) {
    uint32_t c0 = (uint32_t)ctr, c1 = (uint32_t)(ctr >> 32), c2 = 0u, c3 = 0u;
    uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        // one 32 x 32 -> 64-bit product per multiplier (v_mad_u64_u32 gives
        // both halves; separate mul_hi / mul_lo cost twice the multiplies)
        const uint64_t pb = (uint64_t)0xCD9E8D57u * c2, pa = (uint64_t)0xD2511F53u * c0;
        const uint32_t hb = (uint32_t)(pb >> 32), lb = (uint32_t)pb;
        const uint32_t ha = (uint32_t)(pa >> 32), la = (uint32_t)pa;
        c0 = hb ^ c1 ^ k0;
        c2 = ha ^ c3 ^ k1;
        c1 = lb;
        c3 = la;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c0;
}

// Keep test of the dropout mask without the float mapping: u = fp32(fold(x)) *
// 4.6566127342e-10 (fold(x) = x < 0 ? -x - 1 : x on the int32 view) is
// non-decreasing in fold(x), so u > p exactly when fold(x) > T, with T the
// largest fold value whose u is <= p (keep_threshold on the host).
__device__ FA_INLINE inline bool philox_keep(uint64_t seed, uint64_t ctr, uint32_t thresh) {
    const int32_t x = (int32_t)philox_word0(seed, ctr);
    return (uint32_t)(x ^ (x >> 31)) > thresh;
}

// All ones when bit `pos` of x is set, else zero (one sign-extending
// bit-field extract); keep_or_zero(v, m) is v where m is all ones, +0 else.
__device__ FA_INLINE inline uint32_t bit_mask(uint32_t x, int pos) {
    return (uint32_t)((int32_t)(x << (31 - pos)) >> 31);
}
__device__ FA_INLINE inline float keep_or_zero(float v, uint32_t m) {
    return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) & m);
}

__device__ FA_INLINE inline float philox_uniform(uint64_t seed, uint64_t ctr) {
    int32_t x = (int32_t)philox_word0(seed, ctr);
    x = x < 0 ? -x - 1 : x;
    return __fmul_rn((float)x, 4.6566127342e-10f);
}

// ---------------------------------------------------------------------------
// Workgroup-id remap so that consecutive logical tiles land on one XCD.
// Hardware dispatches workgroup L to XCD L % 8; logical id = (L % 8) * per + L / 8
// keeps each XCD on a contiguous run of logical tiles (shared K/V stay in one L2).
__device__ FA_INLINE inline int xcd_remap(int L, int N) {
    const int per = N >> 3;
    const int full = per << 3;
    if (L >= full) return L;
    return (L & 7) * per + (L >> 3);
}

// This workgroup's (slice, tile rank) in a grid of n_tiles tiles per slice
// (a slice is one (batch, head) or (batch, KV head)); rank 0 is a slice's
// longest tile under causal masking.  The logical ids of an XCD (xcd_remap)
// are taken by groups of G slices, and the tiles of a group are dealt
// rank-major: the G rank-0 tiles first, then the G rank-1 tiles, ...  Each
// XCD then picks up workgroups longest first within a group, so its CUs run
// out of work together.  Slice-major (a slice's tiles in a row, longest
// first) leaves the longest tile of the XCD's last slice to start late and
// run alone (measured, causal, outputs unchanged: 4096 tokens x 128 heads
// 4-5% per kernel, 1000-2048 tokens 13-22%; non-causal unchanged).  G
// makes one group about fill the XCD's workgroup slots twice (SLOTS = 32 CUs
// x resident workgroups per CU; measured against once and 4 times), so the
// resident workgroups span few slices (K / V / Q tiles shared through the
// XCD's L2), and a group never spans two XCDs.  With FIT (the kernels pass it
// for causal masking: tiles of one length balance in any order), G is lowered
// (to at most half) to a divisor of the XCD's slices: a small last group ran
// its long tiles after the others had drained (measured, causal, outputs unchanged:
// 2 x 3072 x 32 heads and 3 x 4096 x 16 heads at D = 128, 7-11% per step;
// 2 x 4096 x 24 heads at D = 64, 6%).
// (bid, nblocks: the workgroup's index among the nblocks of its kind, for a
// launch that runs two kinds of workgroups)
template <int SLOTS, bool FIT>
__device__ FA_INLINE inline int2 tile_order(int n_tiles, int bid, int nblocks) {
    const int L = xcd_remap(bid, nblocks);
    const int n_slices = nblocks / n_tiles;
    // groups stay inside one XCD's share of the slices
    const int xcd_slices = max(1, (nblocks >> 3) / n_tiles);
    int G = max(1, min(xcd_slices, (2 * SLOTS + n_tiles - 1) / n_tiles));
    if constexpr (FIT) {
        // the largest group size down to half this target (at most 63 below
        // it) that divides the XCD's slices, so that its last group is as large
        // as the others: lane i tests G - i.  (A scalar search loop here raised
        // the kernels' scalar-register pressure into lane spills inside their
        // tile loops; without FIT no trace of the search is compiled, as even
        // its unused form moved the copy-wave forward's prologue, 1-2% slower.)
        const int lane = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
        const int c = G - lane;
        const bool divides = 2 * c >= G && (int)((unsigned)xcd_slices % (unsigned)max(c, 1)) == 0;
        const unsigned long long hits = __builtin_amdgcn_ballot_w64(divides);
        if (hits) G -= (int)__builtin_ctzll(hits);
    }
    const int per_group = G * n_tiles;
    const int g = L / per_group;
    const int r = L - g * per_group;
    const int gg = min(G, n_slices - g * G);  // the last group may be smaller
    const int rank = r / gg;
    return make_int2(g * G + (r - rank * gg), rank);
}
// On the host: whether tile_order's plain group size leaves an XCD a last
// group smaller than the others, i.e. whether FIT changes it
inline bool host_group_uneven(int slots, int n_tiles, int nblocks) {
    const int per_xcd = (nblocks >> 3) / n_tiles;
    const int xcd_slices = per_xcd > 1 ? per_xcd : 1;
    const int fill = (2 * slots + n_tiles - 1) / n_tiles;
    const int target = fill < 1 ? 1 : (fill < xcd_slices ? fill : xcd_slices);
    return xcd_slices % target != 0;
}
template <int SLOTS, bool FIT>
__device__ FA_INLINE inline int2 tile_order(int n_tiles) {
    return tile_order<SLOTS, FIT>(n_tiles, (int)blockIdx.x, (int)gridDim.x);
}

// (batch, head) of slice s of the B x NH slices: batch-major (s = b NH + h),
// or head-major (s = h B + b) for a kernel that reads a bias shared by the
// batches (batch stride 0): a group of slices (tile_order) then holds batches
// of one head, which read the same bias rows through the XCD's L2
__device__ FA_INLINE inline int2 slice_bh(int s, int NH, int B, bool head_major) {
    return head_major ? make_int2(s % B, s / B) : make_int2(s / NH, s % NH);
}

// ---------------------------------------------------------------------------
// Raw buffer view of the rows [0, min(nvalid, R)) of a tile of R rows in a
// row-strided [rows][D] slice: loads at byte offsets past the last valid row
// return zeros (hardware range check), which zero-fills tail tiles without any
// per-lane branch or select.  The descriptor is rebuilt per tile (base
// advanced to the tile, record count bounded by the tile's rows), so the range
// check never depends on the scalar offset and only tile-local offsets need 32
// bits: the host bounds the byte span of kTileRows rows below 2^31, whatever
// the length of the whole slice.  The byte count is computed without a branch
// (nvalid <= 0 gives 0) so that a tile load does not end a basic block.
template <typename T, int D, int R>
__device__ FA_INLINE inline __amdgpu_buffer_rsrc_t row_buffer(const T* base, int64_t row_stride, int nvalid) {
    const int nv = min(max(nvalid, 0), R);
    const int bytes = ((nv - 1) * (int)row_stride + D) * (int)sizeof(T) * min(nv, 1);
    // dword 3: DATA_FORMAT = 32 (untyped dword access), no swizzle, no stride
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

// Wait for all outstanding vector-memory loads.  Issued once after the
// per-lane register operands (Q, dO, K, V rows, LSE, delta) are loaded, so the
// compiler's wait tracking starts every tile loop with nothing pending and does
// not re-wait for them (together with the next tile's prefetch) each iteration.
__device__ FA_INLINE inline void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// Wait until at most N vector-memory operations of this wave are outstanding
// (they complete in issue order); expcnt and lgkmcnt are not waited for.
template <int N>
__device__ FA_INLINE inline void wait_vmem_below() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// ---------------------------------------------------------------------------
// One 16-byte-per-lane global -> LDS load (buffer_load_dwordx4 ... lds): lane
// l writes LDS bytes [16 l, 16 l + 16) past `lds`, which must be wave-uniform.
// A function of its own: written directly in the kernel templates, the
// builtin made the host pass emit launch stubs only for the first
// instantiation of each kernel (the library then fails to load).
template <typename T>
__device__ FA_INLINE inline void dma_load16(__amdgpu_buffer_rsrc_t rs, T* lds, int byte_offset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 16, byte_offset, 0, 0, 0);
}

// The same 16-byte-per-lane copy issued from inline assembly, for loops that
// order their copies themselves with explicit vmcnt waits.  The compiler does
// not see it as an LDS write, so it does not make the next LDS read of any
// slot wait for every copy in flight (it cannot tell the slots apart), and it
// does not count it in its own vmcnt waits: those can only wait longer than
// needed (vector-memory operations complete in issue order), never shorter.
// The caller waits for the copy (s_waitcnt vmcnt) before any wave reads its
// destination.  `rs` is the buffer descriptor as four wave-uniform dwords,
// `lds` the LDS byte address of lane 0's chunk (wave-uniform).
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__device__ FA_INLINE inline void dma_load16_untracked(const u32x4& rs, uint32_t lds, int byte_offset) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen lds"
        :
        : "s"(lds), "v"(byte_offset), "s"(rs)
        : "memory", "m0");
}

// Four-dword descriptor of `bytes` bytes at `base` (wave-uniform), for the
// untracked copies
__device__ FA_INLINE inline u32x4 buffer_words(const void* base, int bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    u32x4 w;
    w[0] = __builtin_amdgcn_readfirstlane((unsigned)a);
    w[1] = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32) & 0xFFFFu);
    w[2] = __builtin_amdgcn_readfirstlane((unsigned)bytes);
    w[3] = 0x00020000u;
    return w;
}

// Four-dword buffer descriptor of the rows [0, min(nvalid, R)) of a tile, as
// row_buffer builds it (raw untyped dword access, no stride, no swizzle).
template <typename T, int D, int R>
__device__ FA_INLINE inline u32x4 row_buffer_words(const T* base, int64_t row_stride, int nvalid) {
    const int nv = min(max(nvalid, 0), R);
    const int bytes = ((nv - 1) * (int)row_stride + D) * (int)sizeof(T) * min(nv, 1);
    return buffer_words(base, bytes);
}

// LDS byte address of a __shared__ object (an address-space cast, then the
// 32-bit LDS offset)
__device__ FA_INLINE inline uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// ---------------------------------------------------------------------------
// Direct global -> LDS copy of a [R][D] tile (buffer_load_dwordx4 ... lds):
// no staging registers and no LDS store instructions.  The tile occupies LDS
// rows of W elements (W - D of padding).  One wave instruction writes 64
// consecutive 16-byte LDS chunks, lane l to chunk l (checked on gfx950), so
// LDS chunk c of the tile is row c / CW, column chunk c % CW (CW = W * size /
// 16); padding chunks get an out-of-range offset (they read nothing and land
// as zeros).  Instructions
// are dealt round-robin to the NW waves of the workgroup.  Rows >= nvalid are
// outside the buffer range and land as zeros.  The data is in LDS once the
// issuing wave's vmcnt reaches zero; a workgroup barrier after that wait
// publishes it to the other waves.
template <typename T, int R, int D, int W, int NW>
struct DmaTile {
    static constexpr int EPC = 16 / (int)sizeof(T);
    static constexpr int CD = D / EPC;
    static constexpr int CW = W / EPC;
    static_assert(D % EPC == 0 && W % EPC == 0 && W >= D, "16-byte chunked rows");
    static constexpr int CHUNKS = R * CW;
    static constexpr int NI = (CHUNKS + 63) / 64;
    static constexpr int PER = (NI + NW - 1) / NW;
    int off[PER];
    int wave;

    // wave_id must be wave-uniform (readfirstlane): it selects the LDS
    // destination, which the hardware takes from a scalar register (M0).
    __device__ FA_INLINE inline void init(int64_t row_stride, int lane, int wave_id) {
        wave = wave_id;
#pragma unroll
        for (int t = 0; t < PER; ++t) {
            const int c = 64 * (wave + NW * t) + lane;
            const int row = c / CW, col = c % CW;
            // padding chunks of an LDS row read nothing (out of the buffer's range)
            off[t] = col < CD ? (row * (int)row_stride + col * EPC) * (int)sizeof(T) : kOffNowhere;
        }
    }
    __device__ FA_INLINE inline void load(const T* base, int64_t row_stride, int nvalid, T* lds, int lane) const {
        const __amdgpu_buffer_rsrc_t rs = row_buffer<T, D, R>(base, row_stride, nvalid);
#pragma unroll
        for (int t = 0; t < PER; ++t) {
            const int g = wave + NW * t;
            if (NI % NW == 0 || g < NI) {
                if (CHUNKS % 64 == 0 || 64 * g + lane < CHUNKS)
                    dma_load16(rs, lds + 64 * g * EPC, off[t]);
            }
        }
    }
    // the same copy, not tracked by the compiler (see dma_load16_untracked):
    // the caller waits for it (vmcnt) before the barrier that publishes it
    __device__ FA_INLINE inline void load_untracked(const T* base, int64_t row_stride, int nvalid, const T* lds,
                                                    int lane) const {
        load_words(row_buffer_words<T, D, R>(base, row_stride, nvalid), lds);
    }
    // the same untracked copy through a caller-built descriptor (whose range
    // ends where the readable data ends; chunks past it land as zeros)
    __device__ FA_INLINE inline void load_words(const u32x4& rs, const T* lds) const {
        static_assert(CHUNKS % 64 == 0, "whole instructions (an idle lane would need its own exec mask)");
        const uint32_t l0 = lds_addr(lds);
#pragma unroll
        for (int t = 0; t < PER; ++t) {
            const int g = wave + NW * t;
            if (NI % NW == 0 || g < NI) dma_load16_untracked(rs, l0 + 64 * 16 * g, off[t]);
        }
    }
};

// Direct global -> LDS copy of a K tile and a V tile ([R][D] each, LDS row
// strides KW and VW), as one list of copy instructions (the K tile's, then the
// V tile's) dealt round-robin to NW waves, so that every wave issues the same
// number of them when NW divides the total (a partial vmcnt wait can then
// leave exactly the newest pair of tiles in flight).  Layout of each tile as in
// DmaTile (64 consecutive 16-byte LDS chunks per instruction, padding chunks
// read nothing, rows >= nvalid land as zeros).
template <typename T, int R, int D, int KW, int VW, int NW>
struct DmaTilePair {
    static constexpr int EPC = 16 / (int)sizeof(T);
    static constexpr int CD = D / EPC;
    static constexpr int CWK = KW / EPC, CWV = VW / EPC;
    static_assert(D % EPC == 0 && KW % EPC == 0 && VW % EPC == 0 && KW >= D && VW >= D, "16-byte chunked rows");
    static_assert((R * CWK) % 64 == 0 && (R * CWV) % 64 == 0, "whole instructions per tile");
    static constexpr int NK = R * CWK / 64;
    static constexpr int NV = R * CWV / 64;
    static constexpr int NI = NK + NV;
    static constexpr int PER = (NI + NW - 1) / NW;
    static constexpr int MIN_PER = NI / NW;  // instructions issued by every wave
    int off[PER];
    int wave;

    __device__ FA_INLINE inline void init(int64_t k_stride, int64_t v_stride, int lane, int wave_id) {
        wave = wave_id;
#pragma unroll
        for (int t = 0; t < PER; ++t) {
            const int g = wave + NW * t;
            const bool is_k = g < NK;
            const int cw = is_k ? CWK : CWV;
            const int c = 64 * (is_k ? g : g - NK) + lane;
            const int row = c / cw, col = c % cw;
            const int64_t st = is_k ? k_stride : v_stride;
            off[t] = col < CD ? (row * (int)st + col * EPC) * (int)sizeof(T) : kOffNowhere;
        }
    }
    // Both tiles, with copies the compiler does not track (see
    // dma_load16_untracked): the caller orders them with explicit vmcnt waits.
    // A tile past the sequence (nvalid <= 0) reads nothing and lands as zeros.
    __device__ FA_INLINE inline void load_untracked(const T* kb, int64_t k_stride, int k_valid, const T* k_lds,
                                                    const T* vb, int64_t v_stride, int v_valid, const T* v_lds) const {
        const u32x4 rk = row_buffer_words<T, D, R>(kb, k_stride, k_valid);
        const u32x4 rv = row_buffer_words<T, D, R>(vb, v_stride, v_valid);
        const uint32_t lk = lds_addr(k_lds), lv = lds_addr(v_lds);
#pragma unroll
        for (int t = 0; t < PER; ++t) {
            const int g = wave + NW * t;
            if (g < NK)
                dma_load16_untracked(rk, lk + 64 * 16 * g, off[t]);
            else if (NI % NW == 0 || g < NI)
                dma_load16_untracked(rv, lv + 64 * 16 * (g - NK), off[t]);
        }
    }
};

// Direct global -> LDS copy of a [R][D] tile where each wave instruction
// copies KR = 64 / CW whole LDS rows (lanes >= KR * CW idle): the lane's
// global offset is the same for every instruction up to a scalar row step, so
// the copy keeps one offset register per lane instead of one per instruction.
// Instructions t = wave, wave + NWAVES, ... (wave-uniform check) cover the
// tile's row groups; rows >= nvalid land as zeros.
template <typename T, int R, int D, int W, int NWAVES>
struct DmaRowGroups {
    static constexpr int EPC = 16 / (int)sizeof(T);
    static constexpr int CD = D / EPC;
    static constexpr int CW = W / EPC;
    static_assert(D % EPC == 0 && W % EPC == 0 && W >= D && CW <= 64, "16-byte chunked rows");
    static constexpr int KR = 64 / CW;              // rows per instruction
    static constexpr int NI = (R + KR - 1) / KR;    // instructions per tile
    static constexpr int PER = (NI + NWAVES - 1) / NWAVES;
    int off;   // byte offset of this lane's chunk within its row group
    int rowl;  // this lane's row within the group (KR for idle lanes)
    int wave;

    __device__ FA_INLINE inline void init(int64_t row_stride, int lane, int wave_id) {
        wave = wave_id;
        rowl = lane < KR * CW ? lane / CW : KR;
        // padding chunks read nothing: an offset past the range stays past it
        // (below 2^32) after the group's row step is added (tiles span < 2^31
        // bytes)
        const int col = lane % CW;
        off = col < CD ? ((lane / CW) * (int)row_stride + col * EPC) * (int)sizeof(T) : kOffNowhere;
    }
    __device__ FA_INLINE inline void load(const T* base, int64_t row_stride, int nvalid, T* lds) const {
        const __amdgpu_buffer_rsrc_t rs = row_buffer<T, D, R>(base, row_stride, nvalid);
#pragma unroll
        for (int t = 0; t < PER; ++t) {
            const int g = wave + NWAVES * t;
            // lanes past the KR rows of the group, and (last group) past row R, idle
            const int rows_here = (R % KR == 0 || g < NI - 1) ? KR : R - (NI - 1) * KR;
            if ((NI % NWAVES == 0 || g < NI) && rowl < rows_here)
                dma_load16(rs, lds + g * KR * W, off + g * KR * (int)row_stride * (int)sizeof(T));
        }
    }
    // the same copy, not tracked by the compiler (see dma_load16_untracked):
    // the caller waits for it (vmcnt) before the barrier that publishes it.
    // Idle lanes (past the group's rows) are switched off by the branch, which
    // masks exec around the assembly.
    __device__ FA_INLINE inline void load_untracked(const T* base, int64_t row_stride, int nvalid, const T* lds) const {
        const u32x4 rs = row_buffer_words<T, D, R>(base, row_stride, nvalid);
        const uint32_t l0 = lds_addr(lds);
#pragma unroll
        for (int t = 0; t < PER; ++t) {
            const int g = wave + NWAVES * t;
            const int rows_here = (R % KR == 0 || g < NI - 1) ? KR : R - (NI - 1) * KR;
            if ((NI % NWAVES == 0 || g < NI) && rowl < rows_here)
                dma_load16_untracked(rs, l0 + g * KR * W * (int)sizeof(T), off + g * KR * (int)row_stride * (int)sizeof(T));
        }
    }
};

// One dword per lane global -> LDS, not tracked by the compiler (see
// dma_load16_untracked): lane l writes LDS bytes [4 l, 4 l + 4) past the LDS
// byte address `lds` (wave-uniform).
__device__ FA_INLINE inline void dma_load4_untracked(const u32x4& rs, uint32_t lds, int byte_offset) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %2, 0 offen lds"
        :
        : "s"(lds), "v"(byte_offset), "s"(rs)
        : "memory", "m0");
}

// One dword per lane global -> LDS (buffer_load_dword ... lds): lane l writes
// LDS bytes [4 l, 4 l + 4) past `lds` (wave-uniform).
template <typename T>
__device__ FA_INLINE inline void dma_load4(__amdgpu_buffer_rsrc_t rs, T* lds, int byte_offset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 4, byte_offset, 0, 0, 0);
}

}  // namespace fa
