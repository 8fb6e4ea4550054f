// Kernel parameter blocks and launcher declarations shared by the host shim
// (fa_abi.cpp) and the per-dtype kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

// Strides are in elements; the d stride is 1 (checked by the host shim).
struct FwdParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    float* mx;  // optional row max of the scaled scores
    int64_t q_sb, q_ss, q_sh;
    int64_t k_sb, k_ss, k_sh;
    int64_t v_sb, v_ss, v_sh;
    int64_t o_sb, o_ss, o_sh;
    int B, Sq, Sk, H, Hkv, group;
    int n_qtiles;
    float scale;       // softmax scale
    float scale_log2;  // scale * log2(e)
    float dropout_p;
    float rp;          // 1 / (1 - dropout_p)
    uint32_t keep_thresh;  // keep_threshold(dropout_p)
    uint64_t seed, offset;
    // optional dropout keep bits written for the backward: kb_w = ceil(Sk/32)
    // words per query row, bit j%32 of word j/32 for key j
    uint32_t* kb;
    int kb_w;
    // optional additive bias (B, H, Sq, Sk) in the input dtype or float32; a
    // zero stride broadcasts that dimension, the key stride is 1
    const void* bias;
    int64_t bias_sb, bias_sh, bias_ss;
    int bias_span;  // bytes of one (batch, head) slice: ((Sq - 1) * ss + Sk) * elem
};

struct BwdParams {
    const void* q;
    const void* k;
    const void* v;
    const void* o;
    const void* dout;
    const float* lse;
    void* dq;
    void* dk;
    void* dv;
    // workspace: per (batch, head) a row of ws_stride = 2 * sq_pad floats,
    // LSE * log2(e) (+inf past Sq) then rowsum(dO * O) (0 past Sq)
    float* lse2;   // = workspace
    float* delta;  // = workspace + sq_pad
    int64_t q_sb, q_ss, q_sh;
    int64_t k_sb, k_ss, k_sh;
    int64_t v_sb, v_ss, v_sh;
    int64_t o_sb, o_ss, o_sh;
    int64_t do_sb, do_ss, do_sh;
    int64_t dq_sb, dq_ss, dq_sh;
    int64_t dk_sb, dk_ss, dk_sh;
    int64_t dv_sb, dv_ss, dv_sh;
    int B, Sq, Sk, H, Hkv, group;
    int sq_pad;     // Sq rounded up to kSqPad
    int ws_stride;  // 2 * sq_pad
    float scale, scale_log2, dropout_p, rp;
    uint32_t keep_thresh;  // keep_threshold(dropout_p)
    uint64_t seed, offset;
    const uint32_t* kb;  // optional keep bits from the forward (as in FwdParams)
    int kb_w;
    const void* bias;  // as in FwdParams
    int64_t bias_sb, bias_sh, bias_ss;
    int bias_span;
    void* dbias;       // optional (B, H, Sq, Sk) gradient of the bias, key stride 1
    int64_t dbias_sb, dbias_sh, dbias_ss;  // query stride >= Sk
    int dbias_span;    // bytes of one (batch, head) slice
    int dbias_dtype;   // 0 fp16, 1 bf16, 2 fp32 (the FA_DTYPE_* codes)
    int dbias_es;      // its element size in bytes
    // causal: who writes the zeros of the gradient that no kernel visits
    // (entries above the dK/dV blocks' first query tiles): 0 nobody (the
    // summed form, whose reduction writes them), 1 dkdv_kernel, element by
    // element, 2 the dQ pass that reads dS (dq_from_ds), whole row tails, 3
    // dbias_zero_tails_kernel (the same row tails, on a stream of their own
    // beside the dK/dV pass)
    int dbias_zero_fill;
    // 1: the dQ pass reads dS from dbias (written by the dK/dV pass, dbias_es
    // bytes per element: the input dtype or float32) instead of recomputing
    // it; the gradient's base and row / batch / head strides are then 16-byte
    // aligned and Sk * dbias_es is a multiple of 16
    int dq_from_ds;
    int ds_span;  // readable bytes of one (batch, head) dS slice (dq_from_ds)
    // 1 (set by the launcher, 16-bit inputs): the dQ pass runs first and
    // computes LSE * log2 e and delta of its query rows itself, writing the
    // workspace rows the dK/dV pass then reads (no delta pre-pass)
    int dq_delta;
};

// Sum of per-(batch, head) dBias slices over broadcast dimensions:
// out[bo][ho][i][j] = sum of part[b][h][i][j] over b (sum_b) / h (sum_h);
// part is contiguous (B, H, Sq, SkP) with SkP = Sk rounded up to 4; causal
// entries (j > i) are written as 0 without being read (the dK/dV kernel
// leaves the parts of skipped query tiles unwritten).
struct DbiasReduceParams {
    const void* part;
    int part_dtype;  // 0 fp16, 1 bf16, 2 fp32
    void* out;
    int out_dtype;  // 0 fp16, 1 bf16, 2 fp32
    int64_t out_sb, out_sh, out_ss;
    int B, H, Sq, Sk, SkP;
    int sum_b, sum_h, causal;
};

// per-(batch, head) rows of the backward workspace are padded to a multiple
// of this many queries, so query tiles read whole rows without range checks
constexpr int kSqPad = 128;

// Largest fold value x in [0, 2^31) whose uniform fp32(x) * 4.6566127342e-10
// (round to nearest, as the device computes it) is <= p: a mask element is
// kept exactly when its fold value exceeds it (host code, fa_abi.cpp).
uint32_t keep_threshold(float p);

// dtype-specific launchers, one translation unit per pass (fwd / bwd):
// fa_{fwd,bwd}_{bf16,f16,f32}.hip without a bias, fa_{fwd,bwd}_bias_{bf16,f16,f32}.hip
// with a bias of the input dtype, fa_{fwd,bwd}_bias32_{bf16,f16}.hip with a float32 bias
hipError_t launch_fwd_bf16(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s);
hipError_t launch_fwd_f16(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s);
hipError_t launch_fwd_f32(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s);
hipError_t launch_fwd_bias_bf16(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s);
hipError_t launch_fwd_bias_f16(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s);
hipError_t launch_fwd_bias_f32(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s);
hipError_t launch_fwd_bias32_bf16(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s);
hipError_t launch_fwd_bias32_f16(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s);
// stage: 0 = delta pre-pass, 1 = dK/dV, 2 = dQ, 3 = the workspace rows and dQ
// (a recomputing dQ pass), -1 = the whole backward (3 then 1, or 0, 1, 2 when
// dQ reads the dS of the dK/dV pass)
hipError_t launch_bwd_bf16(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s);
hipError_t launch_bwd_f16(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s);
hipError_t launch_bwd_f32(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s);
hipError_t launch_bwd_bias_bf16(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s);
hipError_t launch_bwd_bias_f16(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s);
hipError_t launch_bwd_bias_f32(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s);
hipError_t launch_bwd_bias32_bf16(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s);
hipError_t launch_bwd_bias32_f16(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s);
// head dim 256, 16-bit inputs without a bias: fa_{fwd,bwd}_d256_{bf16,f16}.hip
// (D must be 256; the argument keeps the signature of the other launchers)
hipError_t launch_fwd_d256_bf16(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s);
hipError_t launch_fwd_d256_f16(const FwdParams& p, int D, bool causal, bool dropout, hipStream_t s);
hipError_t launch_bwd_d256_bf16(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s);
hipError_t launch_bwd_d256_f16(const BwdParams& p, int D, bool causal, bool dropout, int stage, hipStream_t s);
// fa_misc.hip
hipError_t launch_dropout_mask(uint64_t seed, uint64_t offset, int B, int H, int Sq, int Sk, float p,
                               uint8_t* keep, hipStream_t s);
hipError_t launch_rand(uint64_t seed, const uint64_t* ctr, int64_t n, float* u, hipStream_t s);
// the forward's dropout keep bits (p.kb, p.kb_w, seed, offset, keep_thresh),
// for the B*H*Sq rows of p; with causal, words whose keys all follow the query
// may be left unwritten
hipError_t launch_keep_bits(const FwdParams& p, bool causal, hipStream_t s);
hipError_t launch_dbias_reduce(const DbiasReduceParams& r, hipStream_t s);
// the causal dBias zeros of dbias_zero_fill == 2 / 3 (dq_from_ds): for each
// 128-query tile, keys from the tile's end on
hipError_t launch_dbias_zero_tails(const BwdParams& p, hipStream_t s);

}  // namespace fa
