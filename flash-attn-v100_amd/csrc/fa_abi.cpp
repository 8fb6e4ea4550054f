// Host side of the C ABI declared in include/fa_abi.h: argument validation
// (pure host code, no HIP call before it passes) and dispatch to the dtype
// launchers.  Launches on the caller's stream and never synchronises.
// Library state, all of it per GPU and created lazily:
//  * a 32 MiB static __device__ scratch (fa_bwd_static's workspace), reserved
//    in every process that loads the library, and its address (looked up once
//    under g_scratch_mu);
//  * only when the environment sets FA_DBIAS_SIDE_STREAM=1: one side stream
//    and two events, on which the whole backward writes the zero tails of a
//    causal bias gradient beside the dK/dV pass; enqueues that use it are
//    serialised by g_side_mu, and it is never used while the caller's stream
//    (or the side stream) is being captured into a graph.
// Without that variable every call is stateless apart from the scratch, and
// re-entrant from any number of threads and streams.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <mutex>

#include "fa_abi.h"
#include "fa_params.hpp"

// Device scratch of fa_bwd_static: the backward workspace for callers that
// cannot allocate.  Each GPU holds its own copy at its own address; host code
// never passes this name to a kernel or a copy (it is a host-side stand-in),
// only the address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[FA_BWD_STATIC_SCRATCH_BYTES];

namespace fa {

// Largest fold value x with fp32(x) * 4.6566127342e-10 <= p, by bisection over
// the same int -> float conversion and fp32 multiply the device performs
// (u is non-decreasing in x).
uint32_t keep_threshold(float p) {
    auto u = [](uint32_t x) {
        volatile float xf = (float)(int32_t)x;  // the device's int -> float conversion, then one fp32 multiply
        return xf * 4.6566127342e-10f;
    };
    uint32_t lo = 0, hi = 0x7fffffffu;  // u(lo) = 0 <= p; u(hi) ~ 1 > p for p < 1
    if (!(u(hi) > p)) return hi;
    while (hi - lo > 1) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (u(mid) <= p)
            lo = mid;
        else
            hi = mid;
    }
    return lo;
}

}  // namespace fa

namespace {

// device address of `scratch` per GPU, looked up on the first fa_bwd_static
// call on that GPU
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// the stream's device (the current one for the null stream); its scratch
// address, looked up with that device current; nullptr on any HIP error
void* static_scratch(hipStream_t s) {
    int dev = -1, cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return nullptr;
    dev = cur;
    if (s != nullptr) {
        hipDevice_t d;
        if (hipStreamGetDevice(s, &d) != hipSuccess) return nullptr;
        dev = (int)d;
    }
    if (dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev]) return g_scratch_ptr[dev];
    if (dev != cur && hipSetDevice(dev) != hipSuccess) return nullptr;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    if (e != hipSuccess || ptr == nullptr) return nullptr;
    g_scratch_ptr[dev] = ptr;
    return ptr;
}

// A library-owned stream per GPU (default priority, non-blocking) with a fork
// and a join event, for work of fa_bwd that runs beside the caller's stream
// (opt-in, FA_DBIAS_SIDE_STREAM=1): created on first use with that GPU
// current; nullptr if any HIP call fails.  The caller holds g_side_mu from the
// fork to its join.
struct SideStream {
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    bool tried = false;
};
std::mutex g_side_mu;
SideStream g_side[kMaxDevices];

int stream_device(hipStream_t s) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return -1;
    if (s == nullptr) return cur;
    hipDevice_t d;
    if (hipStreamGetDevice(s, &d) != hipSuccess) return -1;
    return (int)d;
}

SideStream* side_stream(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return nullptr;
    SideStream& ss = g_side[dev];
    if (ss.tried) return ss.s ? &ss : nullptr;
    ss.tried = true;
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return nullptr;
    if (dev != cur && hipSetDevice(dev) != hipSuccess) return nullptr;
    hipStream_t st = nullptr;
    hipEvent_t ef = nullptr, ej = nullptr;
    bool ok = hipStreamCreateWithFlags(&st, hipStreamNonBlocking) == hipSuccess &&
              hipEventCreateWithFlags(&ef, hipEventDisableTiming) == hipSuccess &&
              hipEventCreateWithFlags(&ej, hipEventDisableTiming) == hipSuccess;
    if (dev != cur) (void)hipSetDevice(cur);
    if (!ok) {
        if (ej) (void)hipEventDestroy(ej);
        if (ef) (void)hipEventDestroy(ef);
        if (st) (void)hipStreamDestroy(st);
        (void)hipGetLastError();
        return nullptr;
    }
    ss.s = st;
    ss.fork = ef;
    ss.join = ej;
    return &ss;
}

// FA_DBIAS_SIDE_STREAM=1 in the environment (read at each call)
bool side_stream_wanted() {
    const char* v = std::getenv("FA_DBIAS_SIDE_STREAM");
    return v != nullptr && v[0] == '1' && v[1] == '\0';
}

// whether a stream is being captured into a graph (true on a query error too:
// then the side stream is not used)
bool capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) {
        (void)hipGetLastError();
        return true;
    }
    return st != hipStreamCaptureStatusNone;
}

int elem_size(int32_t dtype) { return dtype == FA_DTYPE_F32 ? 4 : 2; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Strides beyond 2^40 elements (larger than any device memory) are refused
// before any arithmetic on them, so that the products below stay far from
// int64 overflow.
constexpr int64_t kMaxStride = (int64_t)1 << 40;

// a * b for non-negative a, b; -1 when the product exceeds 2^62
int64_t mul_capped(int64_t a, int64_t b) {
    int64_t r;
    if (__builtin_mul_overflow(a, b, &r) || r > ((int64_t)1 << 62)) return -1;
    return r;
}

// d stride 1; b, s, h strides non-negative multiples of 16 bytes
int32_t check_strides(const int64_t st[4], int es) {
    if (st[3] != 1) return FA_ERR_STRIDE;
    for (int i = 0; i < 3; ++i) {
        if (st[i] < 0) return FA_ERR_STRIDE;
        if (st[i] > kMaxStride) return FA_ERR_TOO_LARGE;
        if ((st[i] * es) % 16 != 0) return FA_ERR_STRIDE;
    }
    return FA_OK;
}

int32_t check_common(int32_t B, int32_t Sq, int32_t Sk, int32_t H, int32_t Hkv, int32_t D, int32_t dtype,
                     float scale, float dropout_p) {
    if (B < 0 || Sq < 0 || Sk < 0 || H < 0 || Hkv < 0) return FA_ERR_SHAPE;
    if (dtype != FA_DTYPE_F16 && dtype != FA_DTYPE_BF16 && dtype != FA_DTYPE_F32) return FA_ERR_DTYPE;
    // 256: 16-bit inputs only (and no bias: fa_fwd_check / fa_bwd_check)
    if (D != 32 && D != 64 && D != 128 && !(D == 256 && dtype != FA_DTYPE_F32)) return FA_ERR_HEAD_DIM;
    if (H == 0 || Hkv == 0 || H % Hkv != 0) return FA_ERR_HEADS;
    if (!std::isfinite(scale) || !(scale > 0.f)) return FA_ERR_SCALE;
    if (!std::isfinite(dropout_p) || dropout_p < 0.f || dropout_p >= 1.f) return FA_ERR_DROPOUT;
    // byte offsets within one row of the backward workspace (2 * Sq floats)
    // and of the keep bits stay 32-bit
    if (Sq >= (1 << 28) || Sk >= (1 << 28)) return FA_ERR_TOO_LARGE;
    // grid sizes: (ceil(S / 32) tiles) x heads x batch must fit a 32-bit grid
    // (tiles x heads < 2^54; compared against the limit divided by the batch)
    const int64_t tiles = ((int64_t)(Sq > Sk ? Sq : Sk) + 31) / 32;
    if (B > 0 && tiles * (int64_t)H > 0x7fffffffLL / B) return FA_ERR_TOO_LARGE;
    return FA_OK;
}

void split(const int64_t st[4], int64_t& sb, int64_t& ss, int64_t& sh) {
    sb = st[0];
    ss = st[1];
    sh = st[2];
}

int32_t status_of(hipError_t e) { return e == hipSuccess ? FA_OK : FA_ERR_LAUNCH; }

// The kernels copy tiles of a (batch, head) slice through a buffer descriptor
// rebuilt per tile, whose 32-bit byte range covers at most the tile's rows;
// lanes address up to kTileRows rows past a tile's first row (padding chunks
// sit past the range), so the byte span of kTileRows rows must stay below
// 2^31.  The length of the whole slice is not limited.
constexpr int32_t kTileRows = 256;

int32_t check_span(const int64_t st[4], int32_t S, int32_t D, int es) {
    if (S <= 0) return FA_OK;
    const int64_t span = ((int64_t)(kTileRows - 1) * st[1] + D) * es;
    return span < (1LL << 31) ? FA_OK : FA_ERR_TOO_LARGE;
}

// The kernels address one (batch, head) slice of the bias / its gradient
// through a buffer whose 32-bit offsets are (row * i_stride + key) * elem with
// row < Sq + 256 and key < Sk + 256 (tiles overhang the sequences).
int32_t check_slice_offsets(const int64_t st[4], int32_t Sq, int32_t Sk, int es) {
    if (st[2] > kMaxStride) return FA_ERR_TOO_LARGE;
    const int64_t rows = (int64_t)(Sq > 0 ? Sq : 1) + 256;
    const int64_t span = mul_capped(rows, st[2]);
    return span >= 0 && (span + Sk + 256) * es < (1LL << 31) ? FA_OK : FA_ERR_TOO_LARGE;
}

// bytes of one (batch, head) slice: rows [0, Sq) of Sk keys
int32_t slice_span(const int64_t st[4], int32_t Sq, int32_t Sk, int es) {
    return Sq > 0 ? (int32_t)(((int64_t)(Sq - 1) * st[2] + Sk) * es) : 0;
}

// Optional bias: element type = the input dtype or float32; (b, h, i, j)
// strides, j stride 1, the others non-negative multiples of 16 bytes (zero
// broadcasts), base 16-byte aligned; the kernels read 4 consecutive keys of a
// row with one 8- or 16-byte load.
int32_t check_bias(const void* bias, const int64_t st[4], int32_t bias_dtype, int32_t dtype, int32_t Sq,
                   int32_t Sk) {
    if (!bias) return FA_OK;
    if (bias_dtype != dtype && bias_dtype != FA_DTYPE_F32) return FA_ERR_BIAS;
    const int es = elem_size(bias_dtype);
    if (!aligned16(bias) || st[3] != 1) return FA_ERR_BIAS;
    for (int i = 0; i < 3; ++i) {
        if (st[i] < 0) return FA_ERR_BIAS;
        if (st[i] > kMaxStride) return FA_ERR_TOO_LARGE;
        if ((st[i] * es) % 16 != 0) return FA_ERR_BIAS;
    }
    return check_slice_offsets(st, Sq, Sk, es);
}

// The bias gradient is summed over a dimension whose dbias stride is 0 (batch
// or head, with more than one of them): the dK/dV kernel then writes
// per-(batch, head) parts into the workspace and a reduction kernel sums them.
bool dbias_reduced(const fa_bwd_args* a) {
    return a->dbias && ((a->dbias_stride[0] == 0 && a->batch > 1) || (a->dbias_stride[1] == 0 && a->num_heads > 1));
}
// Element type of the parts: the gradient's own dtype when it is the 16-bit
// input dtype (each part rounded once to it, as the unsummed gradient is; the
// dQ pass then reads its dS at half the bytes), float32 otherwise.
int32_t dbias_part_dtype(const fa_bwd_args* a) {
    return a->dtype != FA_DTYPE_F32 && a->dbias_dtype == a->dtype ? a->dtype : FA_DTYPE_F32;
}
// key row length of the parts: Sk rounded up to whole 16-byte rows
int32_t dbias_part_row(const fa_bwd_args* a) {
    const int32_t per16 = 16 / elem_size(dbias_part_dtype(a));
    return (a->seqlen_k + per16 - 1) / per16 * per16;
}

// Optional bias gradient: dtype fp16, bf16 or fp32; j stride 1, i stride >= Sk
// (rows do not overlap: stores past the last row must leave the slice),
// element-aligned base, non-negative strides.  Summed form: 16-byte aligned
// base and strides that are multiples of 4 (one store of 4 keys).
int32_t check_dbias(const fa_bwd_args* a) {
    const void* dbias = a->dbias;
    const int64_t* st = a->dbias_stride;
    if (!dbias) return FA_OK;
    const int32_t dt = a->dbias_dtype;
    if (dt != FA_DTYPE_F16 && dt != FA_DTYPE_BF16 && dt != FA_DTYPE_F32) return FA_ERR_BIAS;
    const int es = elem_size(dt);
    if (((uintptr_t)dbias % (uintptr_t)es) || st[3] != 1 || st[2] < a->seqlen_k) return FA_ERR_BIAS;
    for (int i = 0; i < 3; ++i) {
        if (st[i] < 0) return FA_ERR_BIAS;
        if (st[i] > kMaxStride) return FA_ERR_TOO_LARGE;
    }
    if (dbias_reduced(a)) {
        if (!aligned16(dbias)) return FA_ERR_BIAS;
        for (int i = 0; i < 3; ++i)
            if (st[i] % 4 != 0) return FA_ERR_BIAS;
        const int pes = elem_size(dbias_part_dtype(a));
        const int64_t part_st[4] = {0, 0, dbias_part_row(a), 1};
        if (check_slice_offsets(part_st, a->seqlen_q, a->seqlen_k, pes)) return FA_ERR_TOO_LARGE;
        // the parts of every (batch, head) must be addressable (and their
        // workspace size representable)
        const int64_t parts = mul_capped(mul_capped((int64_t)a->batch * a->num_heads, a->seqlen_q),
                                         (int64_t)dbias_part_row(a) * pes);
        if (parts < 0) return FA_ERR_TOO_LARGE;
    }
    return check_slice_offsets(st, a->seqlen_q, a->seqlen_k, es);
}

// Backward workspace: B * H rows of 2 * sq_pad float32 (LSE * log2 e, then
// delta), sq_pad = Sq rounded up to kSqPad, rounded up to 256 bytes; then,
// for a summed bias gradient, the (B, H, Sq, Sk rounded up to 16 bytes)
// parts (dbias_part_dtype), rounded up to 256 bytes.
size_t ws_rows_bytes(const fa_bwd_args* a) {
    const size_t sq_pad = ((size_t)a->seqlen_q + fa::kSqPad - 1) / fa::kSqPad * fa::kSqPad;
    const size_t n = (size_t)a->batch * (size_t)a->num_heads * 2 * sq_pad * sizeof(float);
    return (n + 255) & ~(size_t)255;
}
size_t ws_bytes_for(const fa_bwd_args* a) {
    size_t n = ws_rows_bytes(a);
    if (dbias_reduced(a)) {
        const size_t parts = (size_t)a->batch * a->num_heads * a->seqlen_q * dbias_part_row(a) *
                             elem_size(dbias_part_dtype(a));
        n += (parts + 255) & ~(size_t)255;
    }
    return n;
}

}  // namespace

extern "C" {

int32_t fa_abi_version(void) { return FA_ABI_VERSION; }

const char* fa_strerror(int32_t code) {
    switch (code) {
        case FA_OK: return "success";
        case FA_ERR_NULL_ARG: return "a required pointer is NULL";
        case FA_ERR_SHAPE: return "a size is negative or inconsistent";
        case FA_ERR_HEAD_DIM: return "head_dim must be 32, 64 or 128 (or 256 for fp16 / bf16 inputs without a bias)";
        case FA_ERR_DTYPE: return "dtype must be FA_DTYPE_F16, FA_DTYPE_BF16 or FA_DTYPE_F32";
        case FA_ERR_STRIDE: return "the d stride must be 1 and the b/s/h strides multiples of 16 bytes";
        case FA_ERR_HEADS: return "num_heads must be a positive multiple of num_heads_kv";
        case FA_ERR_DROPOUT: return "dropout_p must be in [0, 1)";
        case FA_ERR_WORKSPACE: return "workspace is NULL or smaller than fa_bwd_workspace_size";
        case FA_ERR_ALIGN: return "tensor base pointers must be 16-byte aligned";
        case FA_ERR_SCALE: return "scale must be finite and > 0";
        case FA_ERR_LAUNCH: return "the HIP runtime rejected a kernel launch";
        case FA_ERR_TOO_LARGE: return "problem too large for the kernel grid";
        case FA_ERR_BIAS:
            return "bias needs the input dtype or float32, j stride 1, b/h/i strides multiples of 16 bytes and a "
                   "16-byte aligned base; dbias needs a bias, dtype fp16/bf16/fp32, j stride 1, i stride >= Sk "
                   "and an aligned base";
        case FA_ERR_SCRATCH:
            return "the backward needs more workspace than the static scratch of fa_bwd_static "
                   "(FA_BWD_STATIC_SCRATCH_BYTES); use fa_bwd with a workspace";
        default: return "unknown status code";
    }
}

int32_t fa_fwd_check(const fa_fwd_args* a) {
    if (!a) return FA_ERR_NULL_ARG;
    int32_t st = check_common(a->batch, a->seqlen_q, a->seqlen_k, a->num_heads, a->num_heads_kv, a->head_dim,
                              a->dtype, a->scale, a->dropout_p);
    if (st) return st;
    const int64_t nq = (int64_t)a->batch * a->num_heads * a->seqlen_q;
    if (nq == 0) return FA_OK;
    if (!a->q || !a->o || !a->lse) return FA_ERR_NULL_ARG;
    if (a->seqlen_k > 0 && (!a->k || !a->v)) return FA_ERR_NULL_ARG;
    const int es = elem_size(a->dtype);
    if ((st = check_strides(a->q_stride, es)) || (st = check_strides(a->k_stride, es)) ||
        (st = check_strides(a->v_stride, es)) || (st = check_strides(a->o_stride, es)))
        return st;
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o)) return FA_ERR_ALIGN;
    if (((uintptr_t)a->lse & 3u) || ((uintptr_t)a->max_vals & 3u)) return FA_ERR_ALIGN;
    if ((st = check_span(a->q_stride, a->seqlen_q, a->head_dim, es)) ||
        (st = check_span(a->k_stride, a->seqlen_k, a->head_dim, es)) ||
        (st = check_span(a->v_stride, a->seqlen_k, a->head_dim, es)) ||
        (st = check_span(a->o_stride, a->seqlen_q, a->head_dim, es)))
        return st;
    if ((uintptr_t)a->keep_bits & 3u) return FA_ERR_ALIGN;
    if (a->bias && a->head_dim == 256) return FA_ERR_HEAD_DIM;
    return check_bias(a->bias, a->bias_stride, a->bias_dtype, a->dtype, a->seqlen_q, a->seqlen_k);
}

int32_t fa_fwd(const fa_fwd_args* a, void* stream) {
    int32_t st = fa_fwd_check(a);
    if (st) return st;
    if ((int64_t)a->batch * a->num_heads * a->seqlen_q == 0) return FA_OK;
    fa::FwdParams p{};
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.o = a->o;
    p.lse = a->lse;
    p.mx = a->max_vals;
    split(a->q_stride, p.q_sb, p.q_ss, p.q_sh);
    split(a->k_stride, p.k_sb, p.k_ss, p.k_sh);
    split(a->v_stride, p.v_sb, p.v_ss, p.v_sh);
    split(a->o_stride, p.o_sb, p.o_ss, p.o_sh);
    p.B = a->batch;
    p.Sq = a->seqlen_q;
    p.Sk = a->seqlen_k;
    p.H = a->num_heads;
    p.Hkv = a->num_heads_kv;
    p.group = a->num_heads / a->num_heads_kv;
    p.scale = a->scale;
    p.scale_log2 = a->scale * 1.4426950408889634f;
    p.dropout_p = a->dropout_p;
    p.rp = 1.f / (1.f - a->dropout_p);
    p.keep_thresh = fa::keep_threshold(a->dropout_p);
    p.kb = a->dropout_p > 0.f ? a->keep_bits : nullptr;
    p.kb_w = (a->seqlen_k + 31) / 32;
    p.seed = a->seed;
    p.offset = a->offset;
    p.bias = a->bias;
    p.bias_sb = a->bias_stride[0];
    p.bias_sh = a->bias_stride[1];
    p.bias_ss = a->bias_stride[2];
    p.bias_span = a->bias ? slice_span(a->bias_stride, a->seqlen_q, a->seqlen_k, elem_size(a->bias_dtype)) : 0;
    const bool causal = a->causal != 0;
    const bool dropout = a->dropout_p > 0.f;
    hipStream_t s = (hipStream_t)stream;
    // keep bits requested: draw them first, the forward then reads them
    if (p.kb) {
        const int32_t st = status_of(fa::launch_keep_bits(p, causal, s));
        if (st != FA_OK) return st;
    }
    if (a->bias) {
        const bool b32 = a->bias_dtype == FA_DTYPE_F32;
        switch (a->dtype) {
            case FA_DTYPE_BF16:
                return status_of(b32 ? fa::launch_fwd_bias32_bf16(p, a->head_dim, causal, dropout, s)
                                     : fa::launch_fwd_bias_bf16(p, a->head_dim, causal, dropout, s));
            case FA_DTYPE_F16:
                return status_of(b32 ? fa::launch_fwd_bias32_f16(p, a->head_dim, causal, dropout, s)
                                     : fa::launch_fwd_bias_f16(p, a->head_dim, causal, dropout, s));
            default: return status_of(fa::launch_fwd_bias_f32(p, a->head_dim, causal, dropout, s));
        }
    }
    const bool d256 = a->head_dim == 256;
    switch (a->dtype) {
        case FA_DTYPE_BF16:
            return status_of(d256 ? fa::launch_fwd_d256_bf16(p, a->head_dim, causal, dropout, s)
                                  : fa::launch_fwd_bf16(p, a->head_dim, causal, dropout, s));
        case FA_DTYPE_F16:
            return status_of(d256 ? fa::launch_fwd_d256_f16(p, a->head_dim, causal, dropout, s)
                                  : fa::launch_fwd_f16(p, a->head_dim, causal, dropout, s));
        default: return status_of(fa::launch_fwd_f32(p, a->head_dim, causal, dropout, s));
    }
}

size_t fa_bwd_workspace_size(const fa_bwd_args* a) {
    if (!a) return 0;
    if (check_common(a->batch, a->seqlen_q, a->seqlen_k, a->num_heads, a->num_heads_kv, a->head_dim, a->dtype,
                     a->scale, a->dropout_p))
        return 0;
    return ws_bytes_for(a);
}

int32_t fa_bwd_check(const fa_bwd_args* a, size_t ws_bytes) {
    if (!a) return FA_ERR_NULL_ARG;
    int32_t st = check_common(a->batch, a->seqlen_q, a->seqlen_k, a->num_heads, a->num_heads_kv, a->head_dim,
                              a->dtype, a->scale, a->dropout_p);
    if (st) return st;
    const int64_t nq = (int64_t)a->batch * a->num_heads * a->seqlen_q;
    const int64_t nk = (int64_t)a->batch * a->num_heads_kv * a->seqlen_k;
    if (nq == 0 && nk == 0) return FA_OK;
    if (nq > 0 && (!a->q || !a->o || !a->dout || !a->lse || !a->dq)) return FA_ERR_NULL_ARG;
    if (nk > 0 && (!a->k || !a->v || !a->dk || !a->dv)) return FA_ERR_NULL_ARG;
    const int es = elem_size(a->dtype);
    const int64_t* strides[8] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride,
                                 a->do_stride, a->dq_stride, a->dk_stride, a->dv_stride};
    for (int i = 0; i < 8; ++i)
        if ((st = check_strides(strides[i], es))) return st;
    const void* ptrs[8] = {a->q, a->k, a->v, a->o, a->dout, a->dq, a->dk, a->dv};
    for (int i = 0; i < 8; ++i)
        if (!aligned16(ptrs[i])) return FA_ERR_ALIGN;
    if ((uintptr_t)a->lse & 3u) return FA_ERR_ALIGN;
    const int32_t rows[8] = {a->seqlen_q, a->seqlen_k, a->seqlen_k, a->seqlen_q,
                             a->seqlen_q, a->seqlen_q, a->seqlen_k, a->seqlen_k};
    for (int i = 0; i < 8; ++i)
        if ((st = check_span(strides[i], rows[i], a->head_dim, es))) return st;
    if (a->dbias && !a->bias) return FA_ERR_BIAS;
    if (a->bias && a->head_dim == 256) return FA_ERR_HEAD_DIM;
    if ((uintptr_t)a->keep_bits & 3u) return FA_ERR_ALIGN;
    if ((st = check_bias(a->bias, a->bias_stride, a->bias_dtype, a->dtype, a->seqlen_q, a->seqlen_k)) ||
        (st = check_dbias(a)))
        return st;
    const size_t need = fa_bwd_workspace_size(a);
    if (need > 0 && ws_bytes < need) return FA_ERR_WORKSPACE;
    return FA_OK;
}

}  // extern "C"

namespace {

// fa_bwd_stage; `side` allows the whole backward (stage -1) to write the zero
// tails of a causal bias gradient on the library's side stream
int32_t bwd_run(const fa_bwd_args* a, void* workspace, size_t ws_bytes, int32_t stage, void* stream, bool side) {
    if (stage < -1 || stage > 3) return FA_ERR_SHAPE;
    int32_t st = fa_bwd_check(a, ws_bytes);
    if (st) return st;
    const size_t need = fa_bwd_workspace_size(a);
    if (need > 0 && (!workspace || !aligned16(workspace))) return FA_ERR_WORKSPACE;
    if ((int64_t)a->batch * a->num_heads * a->seqlen_q == 0 &&
        (int64_t)a->batch * a->num_heads_kv * a->seqlen_k == 0)
        return FA_OK;
    fa::BwdParams p{};
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.o = a->o;
    p.dout = a->dout;
    p.lse = a->lse;
    p.dq = a->dq;
    p.dk = a->dk;
    p.dv = a->dv;
    p.sq_pad = (a->seqlen_q + fa::kSqPad - 1) / fa::kSqPad * fa::kSqPad;
    p.ws_stride = 2 * p.sq_pad;
    p.lse2 = (float*)workspace;
    p.delta = (float*)workspace + p.sq_pad;
    split(a->q_stride, p.q_sb, p.q_ss, p.q_sh);
    split(a->k_stride, p.k_sb, p.k_ss, p.k_sh);
    split(a->v_stride, p.v_sb, p.v_ss, p.v_sh);
    split(a->o_stride, p.o_sb, p.o_ss, p.o_sh);
    split(a->do_stride, p.do_sb, p.do_ss, p.do_sh);
    split(a->dq_stride, p.dq_sb, p.dq_ss, p.dq_sh);
    split(a->dk_stride, p.dk_sb, p.dk_ss, p.dk_sh);
    split(a->dv_stride, p.dv_sb, p.dv_ss, p.dv_sh);
    p.B = a->batch;
    p.Sq = a->seqlen_q;
    p.Sk = a->seqlen_k;
    p.H = a->num_heads;
    p.Hkv = a->num_heads_kv;
    p.group = a->num_heads / a->num_heads_kv;
    p.scale = a->scale;
    p.scale_log2 = a->scale * 1.4426950408889634f;
    p.dropout_p = a->dropout_p;
    p.rp = 1.f / (1.f - a->dropout_p);
    p.keep_thresh = fa::keep_threshold(a->dropout_p);
    p.kb = a->dropout_p > 0.f ? a->keep_bits : nullptr;
    p.kb_w = (a->seqlen_k + 31) / 32;
    p.seed = a->seed;
    p.offset = a->offset;
    p.bias = a->bias;
    p.bias_sb = a->bias_stride[0];
    p.bias_sh = a->bias_stride[1];
    p.bias_ss = a->bias_stride[2];
    p.bias_span = a->bias ? slice_span(a->bias_stride, a->seqlen_q, a->seqlen_k, elem_size(a->bias_dtype)) : 0;
    const bool reduce_db = dbias_reduced(a);
    fa::DbiasReduceParams rp{};
    if (reduce_db) {  // parts in the workspace, summed into dbias after dK/dV
        const int SkP = dbias_part_row(a);
        const int32_t pdt = dbias_part_dtype(a);
        const int64_t part_st[4] = {(int64_t)a->num_heads * a->seqlen_q * SkP, (int64_t)a->seqlen_q * SkP, SkP, 1};
        p.dbias = (char*)workspace + ws_rows_bytes(a);
        p.dbias_sb = part_st[0];
        p.dbias_sh = part_st[1];
        p.dbias_ss = part_st[2];
        p.dbias_dtype = pdt;
        p.dbias_es = elem_size(pdt);
        p.dbias_span = slice_span(part_st, a->seqlen_q, a->seqlen_k, p.dbias_es);
        p.dbias_zero_fill = 0;
        rp.part = p.dbias;
        rp.part_dtype = pdt;
        rp.out = a->dbias;
        rp.out_dtype = a->dbias_dtype;
        rp.out_sb = a->dbias_stride[0];
        rp.out_sh = a->dbias_stride[1];
        rp.out_ss = a->dbias_stride[2];
        rp.B = a->batch;
        rp.H = a->num_heads;
        rp.Sq = a->seqlen_q;
        rp.Sk = a->seqlen_k;
        rp.SkP = SkP;
        rp.sum_b = a->dbias_stride[0] == 0 && a->batch > 1;
        rp.sum_h = a->dbias_stride[1] == 0 && a->num_heads > 1;
        rp.causal = a->causal != 0;
    } else {
        p.dbias = a->dbias;
        p.dbias_sb = a->dbias_stride[0];
        p.dbias_sh = a->dbias_stride[1];
        p.dbias_ss = a->dbias_stride[2];
        p.dbias_es = a->dbias ? elem_size(a->dbias_dtype) : 4;
        p.dbias_dtype = a->dbias ? a->dbias_dtype : FA_DTYPE_F32;
        p.dbias_span = a->dbias ? slice_span(a->dbias_stride, a->seqlen_q, a->seqlen_k, p.dbias_es) : 0;
        p.dbias_zero_fill = 1;
    }
    // dQ from the stored dS: 16-bit inputs, dS in their dtype or float32, whole
    // 16-byte chunks (the summed form's parts always qualify: they are in the
    // input dtype or float32, their rows are whole 16-byte chunks, and the
    // readable span covers whole rows)
    p.dq_from_ds = 0;
    p.ds_span = 0;
    if (a->dbias && a->dtype != FA_DTYPE_F32) {
        if (reduce_db) {
            p.dq_from_ds = 1;
            p.ds_span = (int)std::min<int64_t>((int64_t)a->seqlen_q * dbias_part_row(a) * p.dbias_es, 0x7fffffff);
        } else {
            const int64_t es = p.dbias_es;
            const bool chunks = aligned16(a->dbias) && (p.dbias_sb * es) % 16 == 0 && (p.dbias_sh * es) % 16 == 0 &&
                                (p.dbias_ss * es) % 16 == 0 && ((int64_t)a->seqlen_k * es) % 16 == 0;
            if (chunks && (es == 4 || a->dbias_dtype == a->dtype)) {
                p.dq_from_ds = 1;
                p.ds_span = p.dbias_span;
                p.dbias_zero_fill = 2;
            }
        }
    }
    // stage 3 is the dQ pass that recomputes dS; one that reads the dK/dV
    // pass's dS cannot run before it
    if (stage == 3 && p.dq_from_ds) return FA_ERR_SHAPE;
    const bool causal = a->causal != 0;
    const bool dropout = a->dropout_p > 0.f;
    hipStream_t s = (hipStream_t)stream;
    if (a->bias) {
        // The zero tails of a causal gradient written in place (2.15 GB at
        // B=4, H=32, S=4096 bf16) are pure HBM writes.  By default the dQ pass
        // writes them on the caller's stream (dbias_zero_fill 2).  With
        // FA_DBIAS_SIDE_STREAM=1 the whole backward writes them on the side
        // stream while the compute-bound dK/dV pass runs on the caller's,
        // which waits for them (join) before the call returns -- unless either
        // stream is being captured (a stream that joined a capture stays in it
        // until the capture ends, so other calls' work would land in the
        // graph): then the dQ pass writes them as by default.
        std::unique_lock<std::mutex> side_lock(g_side_mu, std::defer_lock);
        SideStream* ss = nullptr;
        bool joined = false;  // the side stream waits on this call's fork
        if (side && stage < 0 && causal && p.dbias_zero_fill == 2 && side_stream_wanted() && !capturing(s)) {
            side_lock.lock();
            ss = side_stream(stream_device(s));
            if (ss && !capturing(ss->s)) {
                hipError_t e = hipEventRecord(ss->fork, s);
                if (e == hipSuccess) e = hipStreamWaitEvent(ss->s, ss->fork, 0);
                if (e == hipSuccess) {
                    joined = true;
                    e = fa::launch_dbias_zero_tails(p, ss->s);
                    if (e == hipSuccess) p.dbias_zero_fill = 3;  // written there; the dQ pass skips them
                }
                (void)hipGetLastError();  // a failed fork falls back to the dQ pass's tails
            }
        }
        const bool b32 = a->bias_dtype == FA_DTYPE_F32;
        const int D = a->head_dim;
        hipError_t e;
        switch (a->dtype) {
            case FA_DTYPE_BF16:
                e = b32 ? fa::launch_bwd_bias32_bf16(p, D, causal, dropout, stage, s)
                        : fa::launch_bwd_bias_bf16(p, D, causal, dropout, stage, s);
                break;
            case FA_DTYPE_F16:
                e = b32 ? fa::launch_bwd_bias32_f16(p, D, causal, dropout, stage, s)
                        : fa::launch_bwd_bias_f16(p, D, causal, dropout, stage, s);
                break;
            default: e = fa::launch_bwd_bias_f32(p, D, causal, dropout, stage, s);
        }
        // the summed gradient follows the dK/dV stage (stream order)
        if (e == hipSuccess && reduce_db && (stage < 0 || stage == 1)) e = fa::launch_dbias_reduce(rp, s);
        // join, whenever the side stream waited on the fork (also after a
        // failed launch: nothing of this call may outlive it on the side
        // stream unordered with the caller's stream)
        if (joined) {
            hipError_t ej = hipEventRecord(ss->join, ss->s);
            if (ej == hipSuccess) ej = hipStreamWaitEvent(s, ss->join, 0);
            if (e == hipSuccess) e = ej;
        }
        return status_of(e);
    }
    const bool d256 = a->head_dim == 256;
    switch (a->dtype) {
        case FA_DTYPE_BF16:
            return status_of(d256 ? fa::launch_bwd_d256_bf16(p, a->head_dim, causal, dropout, stage, s)
                                  : fa::launch_bwd_bf16(p, a->head_dim, causal, dropout, stage, s));
        case FA_DTYPE_F16:
            return status_of(d256 ? fa::launch_bwd_d256_f16(p, a->head_dim, causal, dropout, stage, s)
                                  : fa::launch_bwd_f16(p, a->head_dim, causal, dropout, stage, s));
        default: return status_of(fa::launch_bwd_f32(p, a->head_dim, causal, dropout, stage, s));
    }
}

}  // namespace

extern "C" {

int32_t fa_bwd_stage(const fa_bwd_args* a, void* workspace, size_t ws_bytes, int32_t stage, void* stream) {
    return bwd_run(a, workspace, ws_bytes, stage, stream, true);
}

int32_t fa_bwd(const fa_bwd_args* a, void* workspace, size_t ws_bytes, void* stream) {
    return bwd_run(a, workspace, ws_bytes, -1, stream, true);
}

int32_t fa_bwd_static(const fa_bwd_args* a, void* stream) {
    // everything that can be rejected is rejected before any HIP call
    int32_t st = fa_bwd_check(a, FA_BWD_STATIC_SCRATCH_BYTES);
    if (st == FA_ERR_WORKSPACE) return FA_ERR_SCRATCH;
    if (st) return st;
    if (fa_bwd_workspace_size(a) > FA_BWD_STATIC_SCRATCH_BYTES) return FA_ERR_SCRATCH;
    if ((int64_t)a->batch * a->num_heads * a->seqlen_q == 0 &&
        (int64_t)a->batch * a->num_heads_kv * a->seqlen_k == 0)
        return FA_OK;
    void* ws = static_scratch((hipStream_t)stream);
    if (!ws) return FA_ERR_LAUNCH;
    // one stream only: no library stream or event is created on this path
    return bwd_run(a, ws, FA_BWD_STATIC_SCRATCH_BYTES, -1, stream, false);
}

int32_t fa_dropout_mask(uint64_t seed, uint64_t offset, int32_t B, int32_t H, int32_t Sq, int32_t Sk,
                        float dropout_p, uint8_t* keep, void* stream) {
    if (B < 0 || H < 0 || Sq < 0 || Sk < 0) return FA_ERR_SHAPE;
    if (!std::isfinite(dropout_p) || dropout_p < 0.f || dropout_p >= 1.f) return FA_ERR_DROPOUT;
    // element count, capped (-1) before it could overflow
    const int64_t n = mul_capped(mul_capped((int64_t)B * H, Sq), Sk);
    if (n == 0) return FA_OK;
    if (!keep) return FA_ERR_NULL_ARG;
    if (n < 0 || n > 0x7fffffffLL * 256) return FA_ERR_TOO_LARGE;
    return status_of(fa::launch_dropout_mask(seed, offset, B, H, Sq, Sk, dropout_p, keep, (hipStream_t)stream));
}

int32_t fa_rand(uint64_t seed, const uint64_t* counters, int64_t n, float* u, void* stream) {
    if (n < 0) return FA_ERR_SHAPE;
    if (n == 0) return FA_OK;
    if (!counters || !u) return FA_ERR_NULL_ARG;
    if (n > 0x7fffffffLL * 256) return FA_ERR_TOO_LARGE;
    return status_of(fa::launch_rand(seed, counters, n, u, (hipStream_t)stream));
}

}  // extern "C"
