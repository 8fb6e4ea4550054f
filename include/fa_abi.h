/* C ABI of the MI355X (gfx950) FlashAttention library.
 *
 * Drop-in boundary for the hot path of mini-kio/flash-attn-v100: the Triton
 * launchers that FlashAttentionV100Function calls.  Plain C types only; every
 * buffer is device memory allocated by the caller (the library never
 * allocates).  Work is enqueued on the caller's HIP stream; no call
 * synchronises the host.
 *
 * State held by the library (per GPU, created lazily): fa_bwd_static's
 * device scratch (FA_BWD_STATIC_SCRATCH_BYTES of static __device__ memory,
 * reserved in every process that loads the library) and its looked-up
 * address; and, only when the environment sets FA_DBIAS_SIDE_STREAM=1, one
 * stream and two events on which fa_bwd writes the zero tails of a causal
 * bias gradient (see fa_bwd).  Every entry point may be called from any
 * number of host threads on any streams at once, except that fa_bwd_static
 * calls on one GPU share its scratch (see there).
 *
 * Layout: q, o, dq, dout are (B, Sq, H, D); k, v, dk, dv are (B, Sk, Hkv, D);
 * strides are in ELEMENTS in the order (b, s, h, d); the d stride must be 1,
 * base pointers 16-byte aligned and the b/s/h strides multiples of 16 bytes.
 * lse / max_vals are (B, H, Sq) float32, contiguous.
 * Query head h reads KV head h / (H / Hkv).  Causal masks key j > query i
 * (top-left aligned, also when Sq != Sk).
 *
 * Optional additive bias (NULL = none), logically (B, H, Sq, Sk), element type
 * bias_dtype (the input dtype or FA_DTYPE_F32), strides in ELEMENTS in the
 * order (b, h, i, j): a stride of 0 broadcasts that dimension (the reference's
 * (B|1, H|1, Sq, Sk) shapes); the j stride must be 1, the b/h/i strides
 * multiples of 16 bytes, and the base 16-byte aligned.  It is added in fp32 to
 * the scaled scores before the causal mask (reference
 * forward_kernel.py:166-182).
 *
 * Optional dropout keep bits (NULL = none; ignored when dropout_p == 0): the
 * forward writes the keep mask it applied, and the backward given them reads
 * it instead of regenerating the Philox stream (same mask, same results).
 * keep_bits: 4-byte aligned uint32 words, row ((b*H + h)*Sq + i) of
 * ceil(Sk/32) words, bit j%32 of word j/32 = keep(b, h, i, j); words whose 32
 * keys causal masking removes for query i are left unwritten (the kernels may
 * read them, but their bits never affect a result).
 */
#ifndef FA_ABI_H
#define FA_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 3

/* element types */
#define FA_DTYPE_F16 0
#define FA_DTYPE_BF16 1
#define FA_DTYPE_F32 2

/* status codes (0 = success, negative = error; fa_strerror names them) */
#define FA_OK 0
#define FA_ERR_NULL_ARG -1    /* a required pointer is NULL */
#define FA_ERR_SHAPE -2       /* a size is negative or inconsistent */
#define FA_ERR_HEAD_DIM -3    /* head_dim not in {32, 64, 128}, nor 256 with 16-bit inputs and no bias */
#define FA_ERR_DTYPE -4       /* dtype code not FA_DTYPE_* */
#define FA_ERR_STRIDE -5      /* d stride != 1, or b/s/h stride not a multiple of 16 bytes */
#define FA_ERR_HEADS -6       /* num_heads not a positive multiple of num_heads_kv */
#define FA_ERR_DROPOUT -7     /* dropout_p not in [0, 1) */
#define FA_ERR_WORKSPACE -8   /* workspace NULL or smaller than fa_bwd_workspace_size */
#define FA_ERR_ALIGN -9       /* a tensor base pointer is not 16-byte aligned */
#define FA_ERR_SCALE -10      /* scale not finite and > 0 */
#define FA_ERR_LAUNCH -11     /* the HIP runtime rejected a kernel launch */
#define FA_ERR_TOO_LARGE -12  /* a grid dimension would overflow, or 256 rows of a
                                 tensor (its sequence stride times 256) span >= 2^31
                                 bytes, or Sq + 256 rows of a bias / dbias slice do */
#define FA_ERR_BIAS -13       /* bias / dbias dtype, strides or alignment violate the rules above */
#define FA_ERR_SCRATCH -14    /* fa_bwd_static: the problem needs more workspace than
                                 FA_BWD_STATIC_SCRATCH_BYTES */

/* Size of the device scratch fa_bwd_static uses instead of a workspace
 * argument (one copy per GPU, held until the process ends). */
#define FA_BWD_STATIC_SCRATCH_BYTES (32u << 20)

/* Forward arguments.
 * Replaces the launcher flash_attention_forward_triton_enhanced
 * (kernels/forward_kernel.py:246-387) and its autotuned twin
 * (kernels/forward_kernel.py:445-512), which FlashAttentionV100Function.forward
 * calls at ops/attention.py:182-194.  Differences from the reference, all
 * deliberate: lse is the true natural-log logsumexp of the scaled, masked
 * scores (the reference stored the row sum there, forward_kernel.py:242);
 * max_vals is the row max of the scaled scores, as there (:243); the dropout
 * seed/offset are arguments instead of a device draw plus .item() host sync
 * (:309-311). */
typedef struct fa_fwd_args {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;      /* required */
    float* max_vals; /* optional (NULL = not written) */
    int64_t q_stride[4];
    int64_t k_stride[4];
    int64_t v_stride[4];
    int64_t o_stride[4];
    int32_t batch;
    int32_t seqlen_q;
    int32_t seqlen_k;
    int32_t num_heads;
    int32_t num_heads_kv;
    int32_t head_dim;
    int32_t dtype;
    int32_t causal;
    float scale;
    float dropout_p;
    uint64_t seed;
    uint64_t offset;
    const void* bias;        /* optional additive bias (NULL = none), see the file comment */
    int64_t bias_stride[4];  /* (b, h, i, j) in elements */
    int32_t bias_dtype;      /* dtype, or FA_DTYPE_F32 */
    uint32_t* keep_bits;     /* optional dropout keep bits out, see the file comment */
} fa_fwd_args;

/* Backward arguments.
 * Replaces flash_attention_backward_triton_enhanced
 * (kernels/backward_kernel.py:208-318), called by
 * FlashAttentionV100Function.backward at ops/attention.py:288-294.  It reads
 * the saved (q, k, v, o, lse) plus the dropout seed/offset of the forward
 * (the reference dropped them, ops/attention.py:209-227) and writes dq, dk,
 * dv in the input dtype (fully overwritten, no zero-init needed).  With a
 * bias, the forward's bias is passed again; if dbias is non-NULL the kernels
 * also write dS = d loss / d(scaled score + bias) into it, logically
 * (B, H, Sq, Sk) with its own (b, h, i, j) strides, as element type
 * dbias_dtype (computed in float32, rounded once) (the reference returned
 * zeros, ops/attention.py:297-301).  A zero b or h stride of dbias sums the
 * gradient over that dimension (the gradient of a bias broadcast over it):
 * the workspace then also holds the per-(b, h) parts (in dbias_dtype when it
 * is the 16-bit input dtype, each part rounded once and the parts summed in
 * float32; float32 parts otherwise), and dbias needs a 16-byte aligned base
 * and strides that are multiples of 4. */
typedef struct fa_bwd_args {
    const void* q;
    const void* k;
    const void* v;
    const void* o;
    const void* dout;
    const float* lse;
    void* dq;
    void* dk;
    void* dv;
    int64_t q_stride[4];
    int64_t k_stride[4];
    int64_t v_stride[4];
    int64_t o_stride[4];
    int64_t do_stride[4];
    int64_t dq_stride[4];
    int64_t dk_stride[4];
    int64_t dv_stride[4];
    int32_t batch;
    int32_t seqlen_q;
    int32_t seqlen_k;
    int32_t num_heads;
    int32_t num_heads_kv;
    int32_t head_dim;
    int32_t dtype;
    int32_t causal;
    float scale;
    float dropout_p;
    uint64_t seed;
    uint64_t offset;
    const void* bias;         /* optional, as in fa_fwd_args */
    int64_t bias_stride[4];
    int32_t bias_dtype;
    void* dbias;              /* optional (B, H, Sq, Sk) gradient of the bias, fully written */
    int64_t dbias_stride[4];  /* (b, h, i, j) in elements; j stride 1, i stride >= Sk; b, h: 0 = sum */
    int32_t dbias_dtype;      /* FA_DTYPE_* of dbias */
    const uint32_t* keep_bits;  /* optional: the forward's dropout keep bits (file comment) */
} fa_bwd_args;

/* Library ABI version (FA_ABI_VERSION).  No reference counterpart. */
int32_t fa_abi_version(void);

/* Static text for a status code.  No reference counterpart (the reference
 * raised Python exceptions, utils.py:57-139). */
const char* fa_strerror(int32_t code);

/* Validate-only: returns the status fa_fwd would return for these arguments
 * without launching anything (host-only; usable without a GPU). */
int32_t fa_fwd_check(const fa_fwd_args* args);

/* Forward: o, lse (and max_vals if non-NULL).  Replaces
 * kernels/forward_kernel.py:246-387 (launch at :349-385). */
int32_t fa_fwd(const fa_fwd_args* args, void* hip_stream);

/* Bytes of device workspace fa_bwd needs: B * H rows of 2 * sq_pad float32
 * (sq_pad = Sq rounded up to 128; LSE * log2 e then delta = rowsum(dO * O),
 * written by the pre-pass), rounded up to 256 bytes; plus, for a summed
 * dbias, B * H * Sq * Skp parts (dbias_dtype when it is the 16-bit input
 * dtype, Skp = Sk rounded up to 8; float32 otherwise, Skp = Sk rounded up to
 * 4), rounded up to 256 bytes; 0 on invalid arguments.
 * The reference had no workspace (it recomputed delta per tile pair,
 * backward_kernel.py:119-121). */
size_t fa_bwd_workspace_size(const fa_bwd_args* args);

/* Validate-only counterpart of fa_bwd (host-only). */
int32_t fa_bwd_check(const fa_bwd_args* args, size_t workspace_bytes);

/* Backward: dq, dk, dv.  Replaces kernels/backward_kernel.py:208-318
 * (launch at :279-316).  workspace: >= fa_bwd_workspace_size bytes,
 * 256-byte aligned device memory.  Stream-ordered on hip_stream.  With a
 * causal bias gradient written in place (16-bit inputs, dS read back by the
 * dQ pass), the zeros above each 128-query tile are written by the dQ pass on
 * hip_stream.  Opt-in (environment FA_DBIAS_SIDE_STREAM=1, read at each
 * call): a small kernel writes them instead on a stream the library owns (one
 * per GPU, default priority, created on first use), forked from hip_stream at
 * entry and joined back to it before return, so that they overlap the dK/dV
 * pass; callers see the same ordering as for any single-stream call.  The
 * side stream is not used while hip_stream (or the side stream) is being
 * captured into a graph, nor by fa_bwd_stage's single stages or by
 * fa_bwd_static; host-side enqueues that use it are serialised by a mutex. */
int32_t fa_bwd(const fa_bwd_args* args, void* workspace, size_t workspace_bytes, void* hip_stream);

/* One stage of fa_bwd: 0 = delta pre-pass (writes the workspace), 1 = dK/dV,
 * 2 = dQ, 3 = the workspace rows and dQ in one pass (16-bit inputs: the dQ
 * kernel computes delta itself; fp32: stage 0 then stage 2); -1 = the whole
 * backward (same as fa_bwd: stage 3 then stage 1, or 0, 1, 2 when dQ reads
 * dS, below).  Without a bias gradient, stages 1 and 2 only read the
 * workspace and are independent of each other, so after stage 0 a caller may
 * run them on two streams; stage 1 after stage 3 gives the same results.
 * (Since ABI version 3: in version 2 stages 1 and 2 were independent after
 * stage 0 in every case.)
 * With one (dbias non-NULL) and 16-bit inputs, stage 1 writes dS (into dbias,
 * or into the workspace for a gradient summed over broadcast dimensions) and
 * stage 2 computes dQ from it: stage 2 must follow stage 1, and stage 3 is
 * FA_ERR_SHAPE.  No reference counterpart (the reference had one fused Triton
 * backward, kernels/backward_kernel.py:17-205). */
int32_t fa_bwd_stage(const fa_bwd_args* args, void* workspace, size_t workspace_bytes, int32_t stage,
                     void* hip_stream);

/* fa_bwd without a workspace argument and without any allocation: the
 * workspace is the library's own device scratch array of
 * FA_BWD_STATIC_SCRATCH_BYTES on the stream's GPU.  Same kernels and results
 * as fa_bwd.  Returns FA_ERR_SCRATCH when fa_bwd_workspace_size(args) exceeds
 * the scratch (B * H * Sq rows up to about 4M, fewer with a summed dbias).
 * Every call on one GPU shares that GPU's scratch: calls that overlap on one
 * GPU (on different streams, or from different threads) race, so a caller
 * serialises them (one stream, or its own ordering).  No scratch contents carry
 * over between calls: stage 0 (or 3) writes every workspace row the later stages read.
 * The first call on a GPU looks the array's device address up once
 * (hipGetSymbolAddress).
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). */
int32_t fa_bwd_static(const fa_bwd_args* args, void* hip_stream);

/* Test hook: the dropout keep mask the kernels apply, keep[b][h][i][j] =
 * U(seed, offset + ((b*H + h)*Sq + i)*Sk + j) > p, as uint8 (B, H, Sq, Sk),
 * from the same device function the forward/backward use.  Counterpart of
 * the tl.rand draw at kernels/forward_kernel.py:198-203 (with the row index
 * i the reference omits restored). */
int32_t fa_dropout_mask(uint64_t seed, uint64_t offset, int32_t batch, int32_t num_heads,
                        int32_t seqlen_q, int32_t seqlen_k, float dropout_p,
                        uint8_t* keep, void* hip_stream);

/* Test hook: u[i] = tl.rand(seed, counters[i]) (Philox4x32-10 word 0 mapped
 * to [0, 1) as Triton does), counters/u in device memory. */
int32_t fa_rand(uint64_t seed, const uint64_t* counters, int64_t n, float* u, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* FA_ABI_H */
