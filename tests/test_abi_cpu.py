"""The C-ABI library on a machine without a GPU: it loads, exports exactly the
functions include/fa_abi.h declares, its structs match the header as compiled
by gcc, and argument validation returns the documented status codes without
any device call."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest
import torch

from flash_attention_v100 import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "fa_abi.h")

CODES = {name: int(val) for name, val in re.findall(r"#define (FA_(?:OK|ERR_\w+))\s+(-?\d+)", open(HEADER).read())}


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(fa_\w+)\s*\(", text, flags=re.M)))


def test_library_loads_and_version():
    lib = _lib.load()
    assert lib.fa_abi_version() == _lib.ABI_VERSION == 3


def test_exports_every_declared_function():
    decl = declared_functions()
    assert set(decl) == set(_lib.EXPORTS), decl
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (fa_\w+)$", out, flags=re.M))
    assert set(decl) <= exported
    lib = _lib.load()
    for name in decl:
        assert hasattr(lib, name)


def test_no_undefined_kernel_symbols():
    # every kernel launch stub the host code references is defined in the library
    out = subprocess.run(["nm", "-D", "--undefined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    missing = [ln.split()[-1] for ln in out.splitlines() if "_ZN2fa" in ln]
    assert not missing, missing


def _c_layout():
    src = r"""
#include <stdio.h>
#include <stddef.h>
#include "fa_abi.h"
#define F(S, m) printf(#S " " #m " %zu\n", offsetof(S, m));
int main(void) {
  printf("fa_fwd_args sizeof %zu\n", sizeof(fa_fwd_args));
  printf("fa_bwd_args sizeof %zu\n", sizeof(fa_bwd_args));
  F(fa_fwd_args, q) F(fa_fwd_args, max_vals) F(fa_fwd_args, q_stride) F(fa_fwd_args, o_stride)
  F(fa_fwd_args, batch) F(fa_fwd_args, causal) F(fa_fwd_args, scale) F(fa_fwd_args, dropout_p)
  F(fa_fwd_args, seed) F(fa_fwd_args, offset) F(fa_fwd_args, bias) F(fa_fwd_args, bias_stride)
  F(fa_fwd_args, bias_dtype) F(fa_fwd_args, keep_bits)
  F(fa_bwd_args, dout) F(fa_bwd_args, lse) F(fa_bwd_args, dv) F(fa_bwd_args, do_stride)
  F(fa_bwd_args, dv_stride) F(fa_bwd_args, batch) F(fa_bwd_args, causal) F(fa_bwd_args, scale)
  F(fa_bwd_args, seed) F(fa_bwd_args, offset) F(fa_bwd_args, bias) F(fa_bwd_args, bias_stride)
  F(fa_bwd_args, bias_dtype) F(fa_bwd_args, dbias) F(fa_bwd_args, dbias_stride) F(fa_bwd_args, dbias_dtype)
  F(fa_bwd_args, keep_bits)
  return 0;
}
"""
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "layout.c")
        exe = os.path.join(d, "layout")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-std=c11", "-I", os.path.dirname(HEADER), c, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    return {tuple(ln.split()[:2]): int(ln.split()[2]) for ln in out.splitlines()}


def test_ctypes_structs_match_header():
    lay = _c_layout()
    assert lay[("fa_fwd_args", "sizeof")] == ctypes.sizeof(_lib.FwdArgs)
    assert lay[("fa_bwd_args", "sizeof")] == ctypes.sizeof(_lib.BwdArgs)
    for (s, m), off in lay.items():
        if m == "sizeof":
            continue
        cls = _lib.FwdArgs if s == "fa_fwd_args" else _lib.BwdArgs
        assert getattr(cls, m).offset == off, (s, m)


def test_integration_stub_struct_matches_header():
    # the ctypes stub a maintainer would copy into the reference must carry every
    # field: a shorter struct makes the library read past its end
    text = open(os.path.join(REPO, "INTEGRATION.md")).read()
    m = re.search(r"class fa_fwd_args\(ctypes.Structure\):.*?_fields_ = (\[.*?\])\s*(?:#[^\n]*)?\n", text, flags=re.S)
    assert m, "stub struct not found"
    fields = eval(m.group(1), {"ctypes": ctypes, "_I64x4": ctypes.c_int64 * 4})
    stub = type("Stub", (ctypes.Structure,), {"_fields_": fields})
    assert ctypes.sizeof(stub) == ctypes.sizeof(_lib.FwdArgs)
    assert [f[0] for f in fields] == [f[0] for f in _lib.FwdArgs._fields_]


def test_strerror_names_every_code():
    for name, code in CODES.items():
        msg = _lib.strerror(code)
        assert msg and msg != "unknown status code", name
    assert _lib.strerror(12345) == "unknown status code"


# ----------------------------------------------------------------------------- validation

def _cpu_fwd(B=2, Sq=64, Sk=64, H=4, Hkv=4, D=64, dtype=torch.float16):
    q = torch.zeros(B, Sq, H, D, dtype=dtype)
    k = torch.zeros(B, Sk, Hkv, D, dtype=dtype)
    v = torch.zeros(B, Sk, Hkv, D, dtype=dtype)
    o = torch.zeros_like(q)
    lse = torch.zeros(B, H, Sq, dtype=torch.float32)
    keep = (q, k, v, o, lse)
    a = _lib.fwd_args(q, k, v, o, lse, None, True, D ** -0.5, 0.0, 0, 0)
    return a, keep


def _status(a):
    return _lib.load().fa_fwd_check(ctypes.byref(a))


def test_fwd_check_accepts_valid():
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        for D in (32, 64, 128):
            a, _ = _cpu_fwd(D=D, dtype=dt)
            assert _status(a) == CODES["FA_OK"]


def test_head_dim_256_only_for_16_bit_inputs_without_bias():
    for dt in (torch.float16, torch.bfloat16):
        a, _ = _cpu_fwd(D=256, dtype=dt)
        assert _status(a) == CODES["FA_OK"]
    a, _ = _cpu_fwd(D=256, dtype=torch.float32)
    assert _status(a) == CODES["FA_ERR_HEAD_DIM"]
    # with a bias (forward and backward checks)
    B, S, H, D = 1, 64, 2, 256
    q = torch.zeros(B, S, H, D, dtype=torch.bfloat16)
    lse = torch.zeros(B, H, S)
    bias = torch.zeros(B, H, S, S, dtype=torch.bfloat16)
    pb = _lib.prepare_bias(bias, B, H, S, S, torch.bfloat16)
    a = _lib.fwd_args(q, q, q, q, lse, None, True, D ** -0.5, 0.0, 0, 0, pb)
    assert _status(a) == CODES["FA_ERR_HEAD_DIM"]
    lib = _lib.load()
    ba = _lib.bwd_args(q, q, q, q, q, lse, q, q, q, True, D ** -0.5, 0.0, 0, 0, pb)
    assert lib.fa_bwd_check(ctypes.byref(ba), 1 << 20) == CODES["FA_ERR_HEAD_DIM"]
    ba = _lib.bwd_args(q, q, q, q, q, lse, q, q, q, True, D ** -0.5, 0.0, 0, 0)
    assert lib.fa_bwd_check(ctypes.byref(ba), lib.fa_bwd_workspace_size(ctypes.byref(ba))) == CODES["FA_OK"]


def test_padded_head_dim_rule():
    assert [_lib.padded_head_dim(d) for d in (1, 32, 33, 64, 65, 128)] == [32, 32, 64, 64, 128, 128]
    assert _lib.padded_head_dim(129) == 0 and _lib.padded_head_dim(256) == 0  # dtype unknown
    for dt in (torch.float16, torch.bfloat16):
        assert _lib.padded_head_dim(129, dt) == 256 and _lib.padded_head_dim(256, dt) == 256
        assert _lib.padded_head_dim(257, dt) == 0 and _lib.padded_head_dim(200, dt, bias=True) == 0
        assert _lib.padded_head_dim(100, dt, bias=True) == 128
    assert _lib.padded_head_dim(200, torch.float32) == 0


@pytest.mark.parametrize("field,value,code", [
    ("head_dim", 96, "FA_ERR_HEAD_DIM"),
    ("head_dim", 512, "FA_ERR_HEAD_DIM"),
    ("head_dim", 192, "FA_ERR_HEAD_DIM"),
    ("dtype", 7, "FA_ERR_DTYPE"),
    ("batch", -1, "FA_ERR_SHAPE"),
    ("seqlen_k", -3, "FA_ERR_SHAPE"),
    ("num_heads_kv", 3, "FA_ERR_HEADS"),
    ("num_heads_kv", 0, "FA_ERR_HEADS"),
    ("dropout_p", 1.0, "FA_ERR_DROPOUT"),
    ("dropout_p", -0.1, "FA_ERR_DROPOUT"),
    ("dropout_p", float("nan"), "FA_ERR_DROPOUT"),
    ("scale", 0.0, "FA_ERR_SCALE"),
    ("scale", -1.0, "FA_ERR_SCALE"),
    ("scale", float("inf"), "FA_ERR_SCALE"),
    ("q", None, "FA_ERR_NULL_ARG"),
    ("lse", None, "FA_ERR_NULL_ARG"),
])
def test_fwd_check_rejects(field, value, code):
    a, _keep = _cpu_fwd()
    setattr(a, field, value)
    assert _status(a) == CODES[code]
    # the launching entry point returns the same code and touches no device
    assert _lib.load().fa_fwd(ctypes.byref(a), None) == CODES[code]


def test_fwd_check_strides_and_alignment():
    a, _keep = _cpu_fwd()
    a.q_stride[3] = 2
    assert _status(a) == CODES["FA_ERR_STRIDE"]
    a, _keep = _cpu_fwd()
    a.k_stride[1] = a.k_stride[1] + 1  # not a multiple of 16 bytes
    assert _status(a) == CODES["FA_ERR_STRIDE"]
    a, _keep = _cpu_fwd()
    a.v = a.v + 2
    assert _status(a) == CODES["FA_ERR_ALIGN"]


def test_fwd_check_accepts_slices_beyond_2_gib():
    # each tile is copied through a buffer range of its own rows, so a (b, h)
    # slice may span more than 2^31 bytes: B=1, S=262144, H=64, D=128 bf16
    # (one slice spans 4 GiB)
    B, S, H, D = 1, 262144, 64, 128
    a, _keep = _cpu_fwd(B=1, Sq=4, Sk=4, H=4, Hkv=4, D=D, dtype=torch.bfloat16)
    a.seqlen_q = a.seqlen_k = S
    a.num_heads = a.num_heads_kv = H
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        setattr(a, name, _lib._I64x4(S * H * D, H * D, D, 1))
    assert ((S - 1) * H * D + D) * 2 >= 2 ** 31
    assert _status(a) == CODES["FA_OK"]
    # the backward checks the same spans
    q = torch.zeros(1, 4, 4, D, dtype=torch.bfloat16)
    lse = torch.zeros(1, 4, 4)
    b = _lib.bwd_args(q, q, q, q, q, lse, q, q, q, True, D ** -0.5, 0.0, 0, 0)
    b.seqlen_q = b.seqlen_k = S
    b.num_heads = b.num_heads_kv = H
    for name in ("q_stride", "k_stride", "v_stride", "o_stride", "do_stride", "dq_stride", "dk_stride", "dv_stride"):
        setattr(b, name, _lib._I64x4(S * H * D, H * D, D, 1))
    ws = _lib.load().fa_bwd_workspace_size(ctypes.byref(b))
    assert _lib.load().fa_bwd_check(ctypes.byref(b), ws) == CODES["FA_OK"]


def test_fwd_check_rejects_tiles_beyond_buffer_range():
    # 256 rows of a tensor must span less than 2^31 bytes (a tile's buffer range)
    a, _keep = _cpu_fwd()
    a.seqlen_k = 300
    a.k_stride[1] = 2 ** 22 + 2 ** 17  # rows 8.25 MiB apart (fp16): 255 row steps exceed 2 GiB
    a.k_stride[0] = a.k_stride[1] * 300
    assert _status(a) == CODES["FA_ERR_TOO_LARGE"]
    a.k_stride[1] = 2 ** 22  # 8 MiB apart: 255 row steps plus one row stay below 2 GiB
    a.k_stride[0] = a.k_stride[1] * 300
    assert _status(a) == CODES["FA_OK"]
    # sequence lengths of 2^28 or more are refused (32-bit workspace offsets)
    a, _keep = _cpu_fwd()
    a.seqlen_k = 2 ** 28
    assert _status(a) == CODES["FA_ERR_TOO_LARGE"]


def test_fwd_check_empty_problem_is_ok():
    a, _keep = _cpu_fwd(Sq=0)
    a.q = None
    assert _status(a) == CODES["FA_OK"]


def test_bwd_workspace_and_checks():
    lib = _lib.load()
    B, S, H, D = 2, 100, 3, 64
    q = torch.zeros(B, S, H, D, dtype=torch.bfloat16)
    lse = torch.zeros(B, H, S)
    a = _lib.bwd_args(q, q, q, q, q, lse, q, q, q, True, 0.125, 0.0, 0, 0)
    ws = lib.fa_bwd_workspace_size(ctypes.byref(a))
    sq_pad = (S + 127) // 128 * 128
    assert ws == ((B * H * 2 * sq_pad * 4 + 255) // 256) * 256
    assert lib.fa_bwd_check(ctypes.byref(a), ws) == CODES["FA_OK"]
    assert lib.fa_bwd_check(ctypes.byref(a), ws - 4) == CODES["FA_ERR_WORKSPACE"]
    assert lib.fa_bwd_stage(ctypes.byref(a), None, ws, 4, None) == CODES["FA_ERR_SHAPE"]
    assert lib.fa_bwd_stage(ctypes.byref(a), None, ws, -2, None) == CODES["FA_ERR_SHAPE"]
    assert lib.fa_bwd(ctypes.byref(a), None, ws, None) == CODES["FA_ERR_WORKSPACE"]
    a.dq = None
    assert lib.fa_bwd_check(ctypes.byref(a), ws) == CODES["FA_ERR_NULL_ARG"]


def test_bwd_static_rejects_problems_beyond_its_scratch():
    # fa_bwd_static validates like fa_bwd and refuses, before any device call,
    # a problem whose workspace exceeds FA_BWD_STATIC_SCRATCH_BYTES
    lib = _lib.load()
    text = open(HEADER).read()
    assert re.search(r"#define FA_BWD_STATIC_SCRATCH_BYTES \(32u << 20\)", text)
    assert _lib.BWD_STATIC_SCRATCH_BYTES == 32 << 20 and _lib.ERR_SCRATCH == CODES["FA_ERR_SCRATCH"]
    q = torch.zeros(1, 8, 64, 64, dtype=torch.bfloat16)
    lse = torch.zeros(1, 64, 8)
    a = _lib.bwd_args(q, q, q, q, q, lse, q, q, q, True, 0.125, 0.0, 0, 0)
    for S, want in ((70000, "FA_ERR_SCRATCH"), (65537, "FA_ERR_SCRATCH")):
        a.seqlen_q = a.seqlen_k = S
        ws = lib.fa_bwd_workspace_size(ctypes.byref(a))
        assert ws > _lib.BWD_STATIC_SCRATCH_BYTES
        assert lib.fa_bwd_static(ctypes.byref(a), None) == CODES[want]
    # exactly at the limit the size check passes (64 heads x 65536 rows x 2 x 4 bytes)
    a.seqlen_q = a.seqlen_k = 65536
    assert lib.fa_bwd_workspace_size(ctypes.byref(a)) == _lib.BWD_STATIC_SCRATCH_BYTES
    # argument errors keep their own codes
    a.dropout_p = 2.0
    assert lib.fa_bwd_static(ctypes.byref(a), None) == CODES["FA_ERR_DROPOUT"]
    a.dropout_p = 0.0
    a.dq = None
    assert lib.fa_bwd_static(ctypes.byref(a), None) == CODES["FA_ERR_NULL_ARG"]
    assert lib.fa_strerror(CODES["FA_ERR_SCRATCH"]).decode().startswith("the backward needs more workspace")


def test_rng_hooks_validation():
    lib = _lib.load()
    assert lib.fa_dropout_mask(1, 0, 1, 1, 4, 4, 1.5, None, None) == CODES["FA_ERR_DROPOUT"]
    assert lib.fa_dropout_mask(1, 0, 1, 1, 4, 4, 0.5, None, None) == CODES["FA_ERR_NULL_ARG"]
    assert lib.fa_dropout_mask(1, 0, 0, 1, 4, 4, 0.5, None, None) == CODES["FA_OK"]
    assert lib.fa_rand(1, None, -1, None, None) == CODES["FA_ERR_SHAPE"]
    assert lib.fa_rand(1, None, 0, None, None) == CODES["FA_OK"]
    assert lib.fa_rand(1, None, 5, None, None) == CODES["FA_ERR_NULL_ARG"]


# ----------------------------------------------------------------------------- bias

def _cpu_bias_fwd(bias_shape=(2, 4, 64, 64), dtype=torch.float16, bias_dtype=None):
    a, keep = _cpu_fwd(dtype=dtype)
    bias = torch.zeros(bias_shape, dtype=bias_dtype or dtype)
    pb = _lib.prepare_bias(bias, 2, 4, 64, 64, dtype)
    a.bias = pb.tensor.data_ptr()
    a.bias_stride = pb.strides
    a.bias_dtype = pb.dtype_code
    return a, (keep, pb)


@pytest.mark.parametrize("shape", [(2, 4, 64, 64), (1, 4, 64, 64), (2, 1, 64, 64), (1, 1, 64, 64), (1, 1, 1, 64)])
def test_bias_check_accepts_broadcast_shapes(shape):
    for dt, bdt in ((torch.float16, None), (torch.bfloat16, torch.float32), (torch.float32, None)):
        a, _keep = _cpu_bias_fwd(shape, dt, bdt)
        assert _status(a) == CODES["FA_OK"], (shape, dt, bdt)


def test_bias_check_rejects():
    a, _keep = _cpu_bias_fwd()
    a.bias_dtype = 1  # bf16 bias with fp16 inputs
    assert _status(a) == CODES["FA_ERR_BIAS"]
    a, _keep = _cpu_bias_fwd()
    a.bias_stride[3] = 2
    assert _status(a) == CODES["FA_ERR_BIAS"]
    a, _keep = _cpu_bias_fwd()
    a.bias_stride[2] = 65  # row stride not a multiple of 16 bytes
    assert _status(a) == CODES["FA_ERR_BIAS"]
    a, _keep = _cpu_bias_fwd()
    a.bias = a.bias + 8
    assert _status(a) == CODES["FA_ERR_BIAS"]


def test_bwd_check_dbias_rules():
    lib = _lib.load()
    B, S, H, D = 2, 100, 3, 64
    q = torch.zeros(B, S, H, D, dtype=torch.bfloat16)
    lse = torch.zeros(B, H, S)
    pb = _lib.prepare_bias(torch.zeros(1, H, S, S, dtype=torch.float32), B, H, S, S, q.dtype)
    db = torch.zeros(B, H, S, S)
    a = _lib.bwd_args(q, q, q, q, q, lse, q, q, q, True, 0.125, 0.0, 0, 0, pb, db)
    ws = lib.fa_bwd_workspace_size(ctypes.byref(a))
    assert lib.fa_bwd_check(ctypes.byref(a), ws) == CODES["FA_OK"]
    a.dbias_stride[3] = 0
    assert lib.fa_bwd_check(ctypes.byref(a), ws) == CODES["FA_ERR_BIAS"]
    a = _lib.bwd_args(q, q, q, q, q, lse, q, q, q, True, 0.125, 0.0, 0, 0, None, db)
    assert lib.fa_bwd_check(ctypes.byref(a), ws) == CODES["FA_ERR_BIAS"]  # dbias without a bias
    a = _lib.bwd_args(q, q, q, q, q, lse, q, q, q, True, 0.125, 0.0, 0, 0, pb, db)
    a.dbias_dtype = 5
    assert lib.fa_bwd_check(ctypes.byref(a), ws) == CODES["FA_ERR_BIAS"]  # unknown dtype
    db16 = torch.zeros(B, H, S, S, dtype=torch.bfloat16)
    a = _lib.bwd_args(q, q, q, q, q, lse, q, q, q, True, 0.125, 0.0, 0, 0, pb, db16)
    assert a.dbias_dtype == _lib.DTYPE_CODES[torch.bfloat16]
    assert lib.fa_bwd_check(ctypes.byref(a), ws) == CODES["FA_OK"]
    a.dbias = a.dbias + 1  # not element-aligned
    assert lib.fa_bwd_check(ctypes.byref(a), ws) == CODES["FA_ERR_BIAS"]


def test_keep_bits_rules():
    lib = _lib.load()
    B, S, H, D = 2, 100, 3, 64
    bits = _lib.alloc_keep_bits(B, H, S, S, "cpu")
    assert bits.shape == (B * H * S, 4) and bits.dtype == torch.int32
    assert _lib.keep_bits_bytes(B, H, S, S) == 4 * bits.numel()
    a, _keep = _cpu_fwd(B=B, Sq=S, Sk=S, H=H, Hkv=H, D=D)
    a.dropout_p = 0.1
    a.keep_bits = bits.data_ptr()
    assert _status(a) == CODES["FA_OK"]
    a.keep_bits = bits.data_ptr() + 2
    assert _status(a) == CODES["FA_ERR_ALIGN"]
    q = torch.zeros(B, S, H, D, dtype=torch.bfloat16)
    lse = torch.zeros(B, H, S)
    a = _lib.bwd_args(q, q, q, q, q, lse, q, q, q, True, 0.125, 0.1, 0, 0, keep_bits=bits)
    ws = lib.fa_bwd_workspace_size(ctypes.byref(a))
    assert lib.fa_bwd_check(ctypes.byref(a), ws) == CODES["FA_OK"]
    a.keep_bits = bits.data_ptr() + 6
    assert lib.fa_bwd_check(ctypes.byref(a), ws) == CODES["FA_ERR_ALIGN"]
    with pytest.raises(ValueError):
        _lib._check_keep_bits(_lib.alloc_keep_bits(B, H, S, S + 40, "cpu"), B, H, S, S, torch.device("cpu"))


@pytest.mark.parametrize("Sk", [1, 32, 96, 4128])
@pytest.mark.parametrize("causal", [False, True])
def test_keep_word_reads_stay_in_the_buffer(Sk, causal):
    """The keep-word reads of the three kernels, restated: every word index
    they form stays below B*H*Sq*kb_w, the buffer the host sizes
    (csrc/fa_fwd.hpp load_kb, csrc/fa_bwd.hpp load_kbits and dq_kernel's
    per-sub-step read, each guarded by key < Sk and query < Sq)."""
    B, H, Sq = 1, 1, 70
    kb_w = (Sk + 31) // 32
    words = B * H * Sq * kb_w
    assert _lib.keep_bits_bytes(B, H, Sq, Sk) == 4 * words
    last = B * H * Sq - 1  # the last (b, h, q) row: its reads end the buffer
    for k0 in range(0, ((Sk + 63) // 64) * 64, 32):  # every 32-key sub-step of every 64-key tile
        if causal and k0 > Sq - 1 + 31:  # waves skip sub-steps past their last query
            continue
        if k0 < Sk:  # the guard: a sub-step that starts past Sk reads no word
            assert last * kb_w + (k0 >> 5) < words
        else:
            assert last * kb_w + (k0 >> 5) >= words  # what an unguarded read would touch


def test_prepare_bias_layout():
    # unaligned rows (Sk = 13 halves = 26 bytes) are copied into 16-byte padded rows
    b = torch.randn(2, 1, 5, 13).to(torch.float16)
    pb = _lib.prepare_bias(b, 2, 3, 5, 13, torch.float16)
    st = list(pb.strides)
    assert st[1] == 0 and st[3] == 1 and (st[2] * 2) % 16 == 0 and (st[0] * 2) % 16 == 0
    assert pb.tensor.data_ptr() % 16 == 0
    assert torch.equal(pb.tensor[:, :, :, :13], b)
    assert pb.shape == (2, 1, 5, 13) and pb.dtype == torch.float16
    # aligned input: used in place
    b2 = torch.randn(1, 3, 5, 16, dtype=torch.float32)
    pb2 = _lib.prepare_bias(b2, 2, 3, 5, 16, torch.bfloat16)
    assert pb2.tensor.data_ptr() == b2.data_ptr() and list(pb2.strides) == [0, 80, 16, 1]
    assert pb2.dtype_code == _lib.DTYPE_CODES[torch.float32]
    # other dtypes are widened to float32; bad shapes raise
    pb3 = _lib.prepare_bias(torch.zeros(1, 1, 5, 16, dtype=torch.float64), 2, 3, 5, 16, torch.float16)
    assert pb3.tensor.dtype == torch.float32
    with pytest.raises(ValueError):
        _lib.prepare_bias(torch.zeros(2, 2, 5, 16), 2, 3, 5, 16, torch.float16)
    # 2-D (Sq, Sk) and 3-D (H, Sq, Sk) biases are the reference validator's
    # shapes (utils.py:204-211); others of those ranks raise
    assert _lib.prepare_bias(torch.zeros(5, 16), 2, 3, 5, 16, torch.float16).shape == (1, 1, 5, 16)
    assert _lib.prepare_bias(torch.zeros(3, 5, 16), 2, 3, 5, 16, torch.float16).shape == (1, 3, 5, 16)
    for bad in [(4, 16), (2, 5, 16), (5,)]:
        with pytest.raises(ValueError):
            _lib.prepare_bias(torch.zeros(*bad), 2, 3, 5, 16, torch.float16)


def test_reduce_dbias_sums_broadcast_dims():
    g = torch.arange(2 * 3 * 4 * 5, dtype=torch.float32).reshape(2, 3, 4, 5)
    pb = _lib.PreparedBias(None, None, 2, (1, 3, 1, 5), torch.bfloat16)
    r = _lib.reduce_dbias(g, pb)
    assert r.shape == (1, 3, 1, 5) and r.dtype == torch.bfloat16
    assert torch.equal(r.float(), g.sum(dim=(0, 2), keepdim=True).to(torch.bfloat16).float())


def test_summed_dbias_workspace_and_rules():
    # a zero batch/head stride of dbias sums the gradient; the workspace then
    # also holds the (B, H, Sq, Sk rounded up to 4) float32 parts of a float32
    # gradient (a gradient in the 16-bit input dtype: below)
    lib = _lib.load()
    B, S, H, D, Sk = 2, 100, 3, 64, 98
    q = torch.zeros(B, S, H, D, dtype=torch.bfloat16)
    k = torch.zeros(B, Sk, H, D, dtype=torch.bfloat16)
    lse = torch.zeros(B, H, S)
    pb = _lib.prepare_bias(torch.zeros(1, H, S, Sk, dtype=torch.bfloat16), B, H, S, Sk, q.dtype)
    full = torch.zeros(B, H, S, Sk)
    a = _lib.bwd_args(q, k, k, q, q, lse, q, k, k, True, 0.125, 0.0, 0, 0, pb, full)
    base = lib.fa_bwd_workspace_size(ctypes.byref(a))
    summed = torch.zeros(1, H, S, 100)[..., :Sk]
    a = _lib.bwd_args(q, k, k, q, q, lse, q, k, k, True, 0.125, 0.0, 0, 0, pb, summed)
    assert list(a.dbias_stride) == [0, S * 100, 100, 1]
    ws = lib.fa_bwd_workspace_size(ctypes.byref(a))
    assert ws == base + ((B * H * S * 100 * 4 + 255) // 256) * 256
    assert lib.fa_bwd_check(ctypes.byref(a), ws) == CODES["FA_OK"]
    assert lib.fa_bwd_check(ctypes.byref(a), base) == CODES["FA_ERR_WORKSPACE"]
    a.dbias_stride[2] = 99  # summed rows must hold 16-byte groups of keys
    assert lib.fa_bwd_check(ctypes.byref(a), ws) == CODES["FA_ERR_BIAS"]
    # a bf16 gradient (the input dtype): bf16 parts, rows of Sk rounded up to 8
    summed16 = torch.zeros(1, H, S, 104, dtype=torch.bfloat16)[..., :Sk]
    a = _lib.bwd_args(q, k, k, q, q, lse, q, k, k, True, 0.125, 0.0, 0, 0, pb, summed16)
    ws16 = lib.fa_bwd_workspace_size(ctypes.byref(a))
    assert ws16 == base + ((B * H * S * 104 * 2 + 255) // 256) * 256
    assert lib.fa_bwd_check(ctypes.byref(a), ws16) == CODES["FA_OK"]
    assert lib.fa_bwd_check(ctypes.byref(a), ws16 - 256) == CODES["FA_ERR_WORKSPACE"]
