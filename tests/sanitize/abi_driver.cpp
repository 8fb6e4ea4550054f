// Drives the C-ABI shim (csrc/fa_abi.cpp), built with host AddressSanitizer and
// UndefinedBehaviorSanitizer against the recording stub launchers, through its
// validation and parameter-building paths: valid calls of every dtype / head
// dim / bias / dropout / dbias form, every rejection, and extreme sizes and
// strides that would overflow careless 32- or 64-bit arithmetic.  Buffers are
// host memory of the exact size: the shim must never dereference them.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "fa_abi.h"
#include "stub_record.h"

static int g_cases = 0, g_fails = 0;
#define CHECK(cond)                                                         \
    do {                                                                    \
        ++g_cases;                                                          \
        if (!(cond)) {                                                      \
            ++g_fails;                                                      \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);     \
        }                                                                   \
    } while (0)

static std::vector<void*> g_bufs;
static void* alloc(size_t bytes) {
    const size_t n = (bytes + 255) / 256 * 256;
    void* p = std::aligned_alloc(256, n ? n : 256);
    std::memset(p, 0, n ? n : 256);
    g_bufs.push_back(p);
    return p;
}

static int esize(int dtype) { return dtype == FA_DTYPE_F32 ? 4 : 2; }

static void contiguous(int64_t st[4], int S, int H, int D) {
    st[0] = (int64_t)S * H * D;
    st[1] = (int64_t)H * D;
    st[2] = D;
    st[3] = 1;
}

static fa_fwd_args make_fwd(int B, int Sq, int Sk, int H, int Hkv, int D, int dtype, int causal, float p = 0.f) {
    fa_fwd_args a;
    std::memset(&a, 0, sizeof(a));
    const int es = esize(dtype);
    a.q = alloc((size_t)B * Sq * H * D * es);
    a.k = alloc((size_t)B * Sk * Hkv * D * es);
    a.v = alloc((size_t)B * Sk * Hkv * D * es);
    a.o = alloc((size_t)B * Sq * H * D * es);
    a.lse = (float*)alloc((size_t)B * H * Sq * 4);
    contiguous(a.q_stride, Sq, H, D);
    contiguous(a.k_stride, Sk, Hkv, D);
    contiguous(a.v_stride, Sk, Hkv, D);
    contiguous(a.o_stride, Sq, H, D);
    a.batch = B;
    a.seqlen_q = Sq;
    a.seqlen_k = Sk;
    a.num_heads = H;
    a.num_heads_kv = Hkv;
    a.head_dim = D;
    a.dtype = dtype;
    a.causal = causal;
    a.scale = 1.f / std::sqrt((float)D);
    a.dropout_p = p;
    a.seed = 42;
    a.bias_stride[3] = 1;
    a.bias_dtype = dtype;
    return a;
}

static fa_bwd_args make_bwd(int B, int Sq, int Sk, int H, int Hkv, int D, int dtype, int causal, float p = 0.f) {
    fa_bwd_args a;
    std::memset(&a, 0, sizeof(a));
    const int es = esize(dtype);
    const size_t nq = (size_t)B * Sq * H * D * es, nk = (size_t)B * Sk * Hkv * D * es;
    a.q = alloc(nq);
    a.k = alloc(nk);
    a.v = alloc(nk);
    a.o = alloc(nq);
    a.dout = alloc(nq);
    a.lse = (const float*)alloc((size_t)B * H * Sq * 4);
    a.dq = alloc(nq);
    a.dk = alloc(nk);
    a.dv = alloc(nk);
    contiguous(a.q_stride, Sq, H, D);
    contiguous(a.k_stride, Sk, Hkv, D);
    contiguous(a.v_stride, Sk, Hkv, D);
    contiguous(a.o_stride, Sq, H, D);
    contiguous(a.do_stride, Sq, H, D);
    contiguous(a.dq_stride, Sq, H, D);
    contiguous(a.dk_stride, Sk, Hkv, D);
    contiguous(a.dv_stride, Sk, Hkv, D);
    a.batch = B;
    a.seqlen_q = Sq;
    a.seqlen_k = Sk;
    a.num_heads = H;
    a.num_heads_kv = Hkv;
    a.head_dim = D;
    a.dtype = dtype;
    a.causal = causal;
    a.scale = 1.f / std::sqrt((float)D);
    a.dropout_p = p;
    a.seed = 7;
    a.bias_stride[3] = 1;
    a.bias_dtype = dtype;
    a.dbias_stride[3] = 1;
    a.dbias_dtype = FA_DTYPE_F32;
    return a;
}

static void fwd_valid() {
    const char* names[3] = {"launch_fwd_f16", "launch_fwd_bf16", "launch_fwd_f32"};
    for (int dt = 0; dt < 3; ++dt)
        for (int D : {32, 64, 128})
            for (int causal = 0; causal < 2; ++causal) {
                fa_fwd_args a = make_fwd(2, 77, 130, 4, 2, D, dt, causal);
                const int before = g_stub.fwd_calls;
                CHECK(fa_fwd_check(&a) == FA_OK);
                CHECK(fa_fwd(&a, nullptr) == FA_OK);
                CHECK(g_stub.fwd_calls == before + 1);
                CHECK(std::strcmp(g_stub.last, names[dt]) == 0);
                CHECK(g_stub.fwd.group == 2 && g_stub.fwd.Sq == 77 && g_stub.fwd.Sk == 130);
                CHECK(g_stub.fwd.kb == nullptr && g_stub.D == D && g_stub.causal == (causal != 0));
                CHECK(std::fabs(g_stub.fwd.scale_log2 - a.scale * 1.4426950408889634f) < 1e-6f);
            }
    // dropout with keep bits: the mask kernel runs first, then the forward reads the bits
    fa_fwd_args a = make_fwd(1, 50, 70, 2, 2, 64, FA_DTYPE_F16, 1, 0.1f);
    a.keep_bits = (uint32_t*)alloc((size_t)1 * 2 * 50 * 3 * 4);
    const int kb = g_stub.keep_bits_calls;
    CHECK(fa_fwd(&a, nullptr) == FA_OK);
    CHECK(g_stub.keep_bits_calls == kb + 1 && g_stub.fwd.kb == a.keep_bits && g_stub.fwd.kb_w == 3);
    CHECK(g_stub.dropout && std::fabs(g_stub.fwd.rp - 1.f / 0.9f) < 1e-6f);
    // keep thresholds are monotone in p and 0 keeps nothing below the smallest draw
    fa_fwd_args b = make_fwd(1, 4, 4, 1, 1, 32, FA_DTYPE_F32, 0, 0.5f);
    CHECK(fa_fwd(&b, nullptr) == FA_OK);
    const uint32_t t5 = g_stub.fwd.keep_thresh;
    CHECK(fa_fwd(&a, nullptr) == FA_OK);
    CHECK(g_stub.fwd.keep_thresh < t5 && t5 < 0x7fffffffu);
    // a float32 bias with bf16 inputs, broadcast over heads
    fa_fwd_args c = make_fwd(2, 40, 33, 3, 3, 128, FA_DTYPE_BF16, 1);
    c.bias = alloc((size_t)2 * 40 * 36 * 4);
    c.bias_dtype = FA_DTYPE_F32;
    c.bias_stride[0] = 40 * 36;
    c.bias_stride[1] = 0;
    c.bias_stride[2] = 36;
    c.bias_stride[3] = 1;
    CHECK(fa_fwd(&c, nullptr) == FA_OK);
    CHECK(std::strcmp(g_stub.last, "launch_fwd_bias32_bf16") == 0);
    CHECK(g_stub.fwd.bias_sh == 0 && g_stub.fwd.bias_span == (39 * 36 + 33) * 4);
    // an empty problem launches nothing
    fa_fwd_args e = make_fwd(0, 10, 10, 2, 2, 64, FA_DTYPE_F16, 0);
    const int n0 = g_stub.fwd_calls;
    CHECK(fa_fwd(&e, nullptr) == FA_OK && g_stub.fwd_calls == n0);
}

static void fwd_rejects() {
    struct Case {
        const char* what;
        int code;
    };
    auto expect = [](fa_fwd_args a, int code) {
        const int before = g_stub.fwd_calls;
        CHECK(fa_fwd_check(&a) == code);
        CHECK(fa_fwd(&a, nullptr) == code);
        CHECK(g_stub.fwd_calls == before);
    };
    fa_fwd_args a = make_fwd(2, 64, 64, 4, 4, 64, FA_DTYPE_F16, 1);
    CHECK(fa_fwd_check(nullptr) == FA_ERR_NULL_ARG);
    fa_fwd_args t = a; t.head_dim = 96; expect(t, FA_ERR_HEAD_DIM);
    t = a; t.dtype = 9; expect(t, FA_ERR_DTYPE);
    t = a; t.batch = -1; expect(t, FA_ERR_SHAPE);
    t = a; t.seqlen_q = INT32_MIN; expect(t, FA_ERR_SHAPE);
    t = a; t.num_heads_kv = 3; expect(t, FA_ERR_HEADS);
    t = a; t.num_heads = 0; expect(t, FA_ERR_HEADS);
    t = a; t.dropout_p = 1.f; expect(t, FA_ERR_DROPOUT);
    t = a; t.dropout_p = NAN; expect(t, FA_ERR_DROPOUT);
    t = a; t.scale = -1.f; expect(t, FA_ERR_SCALE);
    t = a; t.scale = INFINITY; expect(t, FA_ERR_SCALE);
    t = a; t.q = nullptr; expect(t, FA_ERR_NULL_ARG);
    t = a; t.lse = nullptr; expect(t, FA_ERR_NULL_ARG);
    t = a; t.q_stride[3] = 2; expect(t, FA_ERR_STRIDE);
    t = a; t.k_stride[1] += 1; expect(t, FA_ERR_STRIDE);
    t = a; t.v_stride[0] = -64; expect(t, FA_ERR_STRIDE);
    t = a; t.o = (char*)t.o + 2; expect(t, FA_ERR_ALIGN);
    t = a; t.keep_bits = (uint32_t*)((char*)alloc(64) + 2); expect(t, FA_ERR_ALIGN);
    t = a; t.bias = alloc(64 * 64 * 2); t.bias_dtype = FA_DTYPE_BF16; expect(t, FA_ERR_BIAS);
    t = a; t.bias = alloc(64 * 64 * 2); t.bias_stride[2] = 63; expect(t, FA_ERR_BIAS);
    // sizes and strides that overflow careless arithmetic must be refused
    t = a; t.k_stride[1] = (int64_t)1 << 60; expect(t, FA_ERR_TOO_LARGE);
    t = a; t.q_stride[0] = INT64_MAX - 7; expect(t, FA_ERR_TOO_LARGE);
    t = a; t.v_stride[2] = (int64_t)1 << 62; expect(t, FA_ERR_TOO_LARGE);
    t = a; t.batch = INT32_MAX; t.num_heads = t.num_heads_kv = INT32_MAX; t.seqlen_q = t.seqlen_k = 1 << 27;
    expect(t, FA_ERR_TOO_LARGE);
    t = a; t.seqlen_k = 1 << 28; expect(t, FA_ERR_TOO_LARGE);
    t = a; t.bias = alloc(64); t.bias_stride[2] = (int64_t)1 << 61; expect(t, FA_ERR_TOO_LARGE);
    // head dim 256: 16-bit inputs without a bias only, on launchers of its own
    fa_fwd_args w = make_fwd(1, 40, 40, 2, 2, 256, FA_DTYPE_BF16, 1);
    CHECK(fa_fwd(&w, nullptr) == FA_OK);
    CHECK(std::strcmp(g_stub.last, "launch_fwd_d256_bf16") == 0 && g_stub.D == 256);
    w = make_fwd(1, 40, 40, 2, 2, 256, FA_DTYPE_F16, 0);
    CHECK(fa_fwd(&w, nullptr) == FA_OK);
    CHECK(std::strcmp(g_stub.last, "launch_fwd_d256_f16") == 0);
    t = w; t.dtype = FA_DTYPE_F32; expect(t, FA_ERR_HEAD_DIM);
    t = w; t.bias = alloc(40 * 40 * 2); t.bias_dtype = FA_DTYPE_F16; t.bias_stride[1] = 40 * 40; t.bias_stride[2] = 40;
    expect(t, FA_ERR_HEAD_DIM);
    t = w; t.head_dim = 192; expect(t, FA_ERR_HEAD_DIM);
}

static void bwd_paths() {
    fa_bwd_args a = make_bwd(2, 100, 90, 4, 2, 64, FA_DTYPE_BF16, 1);
    const size_t ws = fa_bwd_workspace_size(&a);
    CHECK(ws == (size_t)(2 * 4 * 2 * 128 * 4 + 255) / 256 * 256);
    void* w = alloc(ws);
    CHECK(fa_bwd_check(&a, ws) == FA_OK);
    CHECK(fa_bwd_check(&a, ws - 4) == FA_ERR_WORKSPACE);
    CHECK(fa_bwd(&a, nullptr, ws, nullptr) == FA_ERR_WORKSPACE);
    CHECK(fa_bwd_stage(&a, w, ws, 4, nullptr) == FA_ERR_SHAPE);
    CHECK(fa_bwd_stage(&a, w, ws, -2, nullptr) == FA_ERR_SHAPE);
    CHECK(fa_bwd(&a, w, ws, nullptr) == FA_OK);
    CHECK(std::strcmp(g_stub.last, "launch_bwd_bf16") == 0 && g_stub.stage == -1);
    CHECK(g_stub.bwd.sq_pad == 128 && g_stub.bwd.ws_stride == 256 && g_stub.bwd.group == 2);
    CHECK(g_stub.bwd.lse2 == (float*)w && g_stub.bwd.delta == (float*)w + 128);
    for (int s = 0; s < 4; ++s) {
        CHECK(fa_bwd_stage(&a, w, ws, s, nullptr) == FA_OK);
        CHECK(g_stub.stage == s);
    }
    // head dim 256 (16-bit, no bias) on launchers of its own
    fa_bwd_args a2 = make_bwd(1, 60, 60, 2, 1, 256, FA_DTYPE_F16, 1);
    const size_t ws2 = fa_bwd_workspace_size(&a2);
    CHECK(ws2 > 0 && fa_bwd(&a2, alloc(ws2), ws2, nullptr) == FA_OK);
    CHECK(std::strcmp(g_stub.last, "launch_bwd_d256_f16") == 0 && g_stub.D == 256 && g_stub.stage == -1);
    a2.dtype = FA_DTYPE_F32;
    CHECK(fa_bwd_workspace_size(&a2) == 0 && fa_bwd_check(&a2, ws2) == FA_ERR_HEAD_DIM);
    // a bias gradient summed over the batch: parts in the workspace, then the reduction
    fa_bwd_args b = make_bwd(3, 70, 70, 4, 2, 128, FA_DTYPE_F16, 1);
    b.bias = alloc((size_t)4 * 70 * 72 * 2);
    b.bias_stride[0] = 0;
    b.bias_stride[1] = 70 * 72;
    b.bias_stride[2] = 72;
    b.dbias = alloc((size_t)4 * 70 * 72 * 2);
    b.dbias_dtype = FA_DTYPE_F16;
    b.dbias_stride[0] = 0;
    b.dbias_stride[1] = 70 * 72;
    b.dbias_stride[2] = 72;
    const size_t wsb = fa_bwd_workspace_size(&b);
    const size_t rows = (size_t)(3 * 4 * 2 * 128 * 4 + 255) / 256 * 256;
    // the parts are in the gradient's dtype (fp16, the input dtype): rows of Sk
    // rounded up to 8 elements
    CHECK(wsb == rows + (size_t)(3 * 4 * 70 * 72 * 2 + 255) / 256 * 256);
    const int r0 = g_stub.reduce_calls;
    // dQ reads the stored dS here: it cannot run as the first pass (stage 3)
    CHECK(fa_bwd_stage(&b, alloc(wsb), wsb, 3, nullptr) == FA_ERR_SHAPE);
    CHECK(fa_bwd(&b, alloc(wsb), wsb, nullptr) == FA_OK);
    CHECK(g_stub.reduce_calls == r0 + 1 && g_stub.reduce.sum_b == 1 && g_stub.reduce.sum_h == 0);
    CHECK(g_stub.reduce.SkP == 72 && g_stub.reduce.part_dtype == FA_DTYPE_F16 && g_stub.bwd.dbias_dtype == FA_DTYPE_F16 &&
          g_stub.bwd.dbias_es == 2 && g_stub.bwd.dbias_zero_fill == 0);
    CHECK(std::strcmp(g_stub.last, "launch_bwd_bias_f16") == 0);
    // a causal gradient written in place (dS read back by the dQ pass): the whole
    // backward writes the zero tails on the library's side stream when it can
    // create one; without a device (here) it cannot, and the dQ pass writes them
    fa_bwd_args c = make_bwd(2, 64, 64, 2, 2, 64, FA_DTYPE_BF16, 1);
    c.bias = alloc((size_t)2 * 2 * 64 * 64 * 2);
    c.bias_dtype = FA_DTYPE_BF16;
    c.bias_stride[0] = 2 * 64 * 64;
    c.bias_stride[1] = 64 * 64;
    c.bias_stride[2] = 64;
    c.dbias = alloc((size_t)2 * 2 * 64 * 64 * 2);
    c.dbias_dtype = FA_DTYPE_BF16;
    c.dbias_stride[0] = 2 * 64 * 64;
    c.dbias_stride[1] = 64 * 64;
    c.dbias_stride[2] = 64;
    const size_t wsc = fa_bwd_workspace_size(&c);
    CHECK(fa_bwd(&c, alloc(wsc), wsc, nullptr) == FA_OK);
    CHECK(g_stub.bwd.dq_from_ds == 1 && g_stub.bwd.dbias_zero_fill == 2 && g_stub.stage == -1);
    CHECK(std::strcmp(g_stub.last, "launch_bwd_bias_bf16") == 0);
    // rejections
    fa_bwd_args t = a; t.dq = nullptr; CHECK(fa_bwd_check(&t, ws) == FA_ERR_NULL_ARG);
    t = a; t.dbias = alloc(64); CHECK(fa_bwd_check(&t, ws) == FA_ERR_BIAS);  // dbias without a bias
    t = a; t.dk_stride[1] = (int64_t)1 << 58; CHECK(fa_bwd_check(&t, ws) == FA_ERR_TOO_LARGE);
    t = a; t.dout = (char*)t.dout + 8; CHECK(fa_bwd_check(&t, ws) == FA_ERR_ALIGN);
    CHECK(fa_bwd_workspace_size(nullptr) == 0);
    t = a; t.head_dim = 80; CHECK(fa_bwd_workspace_size(&t) == 0);
    // huge but valid sizes: no overflow in the workspace arithmetic
    t = a; t.batch = 1 << 4; t.num_heads = 1 << 6; t.num_heads_kv = 1 << 6; t.seqlen_q = t.seqlen_k = 1 << 20;
    const size_t big = fa_bwd_workspace_size(&t);
    CHECK(big == (size_t)1 << (4 + 6 + 1 + 20 + 2));
    t.batch = 1 << 12;  // (S / 32) x heads x batch beyond a 32-bit grid: refused, size 0
    CHECK(fa_bwd_workspace_size(&t) == 0 && fa_bwd_check(&t, big) == FA_ERR_TOO_LARGE);
    t.batch = 1 << 4;
    // the no-allocation entry point refuses what its scratch cannot hold, before any device call
    CHECK(fa_bwd_static(&t, nullptr) == FA_ERR_SCRATCH);
    t = a; t.dropout_p = 3.f; CHECK(fa_bwd_static(&t, nullptr) == FA_ERR_DROPOUT);
}

static void misc() {
    for (int c = -20; c <= 2; ++c) CHECK(fa_strerror(c) != nullptr && std::strlen(fa_strerror(c)) > 0);
    CHECK(fa_abi_version() == FA_ABI_VERSION);
    CHECK(fa_dropout_mask(1, 0, 1, 1, 4, 4, 1.5f, nullptr, nullptr) == FA_ERR_DROPOUT);
    CHECK(fa_dropout_mask(1, 0, 1, 1, 4, 4, 0.5f, nullptr, nullptr) == FA_ERR_NULL_ARG);
    CHECK(fa_dropout_mask(1, 0, -1, 1, 4, 4, 0.5f, nullptr, nullptr) == FA_ERR_SHAPE);
    CHECK(fa_dropout_mask(1, 0, INT32_MAX, INT32_MAX, INT32_MAX, INT32_MAX, 0.5f, (uint8_t*)alloc(16), nullptr) ==
          FA_ERR_TOO_LARGE);
    CHECK(fa_rand(1, nullptr, -1, nullptr, nullptr) == FA_ERR_SHAPE);
    CHECK(fa_rand(1, nullptr, 5, nullptr, nullptr) == FA_ERR_NULL_ARG);
    CHECK(fa_rand(1, (const uint64_t*)alloc(16), INT64_MAX, (float*)alloc(16), nullptr) == FA_ERR_TOO_LARGE);
}

int main() {
    fwd_valid();
    fwd_rejects();
    bwd_paths();
    misc();
    for (void* p : g_bufs) std::free(p);
    std::printf("%d checks, %d failed\n", g_cases, g_fails);
    return g_fails ? 1 : 0;
}
