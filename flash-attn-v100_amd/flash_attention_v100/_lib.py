"""ctypes binding of the gfx950 kernel library (``libfa_gfx950.so``).

The library exports the C ABI of ``include/fa_abi.h``.  This module mirrors its
argument structs, loads it (after torch, so that both share torch's HIP
runtime: the library's ``libamdhip64.so.7`` dependency resolves to the copy
torch already loaded) and turns status codes into exceptions.  All memory is
allocated here with torch; the library itself never allocates.

There is no fallback: if the library is missing or fails to load, every entry
point raises :class:`FlashAttentionExtensionError`.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Tuple

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libfa_gfx950.so")
ABI_VERSION = 3
HEAD_DIMS = (32, 64, 128)  # compiled into the kernels for every dtype, with or without a bias
WIDE_HEAD_DIM = 256        # compiled for fp16 / bf16 inputs without a bias
MAX_HEAD_DIM = WIDE_HEAD_DIM

DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}

_I64x4 = ctypes.c_int64 * 4


class FlashAttentionExtensionError(ImportError):
    """The HIP kernel library is missing or unusable (never silently bypassed)."""


class FlashAttentionKernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} failed with status {code}: {message}")
        self.code = code


class FwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p), ("max_vals", ctypes.c_void_p),
        ("q_stride", _I64x4), ("k_stride", _I64x4), ("v_stride", _I64x4), ("o_stride", _I64x4),
        ("batch", ctypes.c_int32), ("seqlen_q", ctypes.c_int32), ("seqlen_k", ctypes.c_int32),
        ("num_heads", ctypes.c_int32), ("num_heads_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("causal", ctypes.c_int32),
        ("scale", ctypes.c_float), ("dropout_p", ctypes.c_float),
        ("seed", ctypes.c_uint64), ("offset", ctypes.c_uint64),
        ("bias", ctypes.c_void_p), ("bias_stride", _I64x4), ("bias_dtype", ctypes.c_int32),
        ("keep_bits", ctypes.c_void_p),
    ]


class BwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("o", ctypes.c_void_p),
        ("dout", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("dq", ctypes.c_void_p), ("dk", ctypes.c_void_p), ("dv", ctypes.c_void_p),
        ("q_stride", _I64x4), ("k_stride", _I64x4), ("v_stride", _I64x4), ("o_stride", _I64x4),
        ("do_stride", _I64x4), ("dq_stride", _I64x4), ("dk_stride", _I64x4), ("dv_stride", _I64x4),
        ("batch", ctypes.c_int32), ("seqlen_q", ctypes.c_int32), ("seqlen_k", ctypes.c_int32),
        ("num_heads", ctypes.c_int32), ("num_heads_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("causal", ctypes.c_int32),
        ("scale", ctypes.c_float), ("dropout_p", ctypes.c_float),
        ("seed", ctypes.c_uint64), ("offset", ctypes.c_uint64),
        ("bias", ctypes.c_void_p), ("bias_stride", _I64x4), ("bias_dtype", ctypes.c_int32),
        ("dbias", ctypes.c_void_p), ("dbias_stride", _I64x4), ("dbias_dtype", ctypes.c_int32),
        ("keep_bits", ctypes.c_void_p),
    ]


EXPORTS = (
    "fa_abi_version", "fa_strerror", "fa_fwd_check", "fa_fwd", "fa_bwd_workspace_size",
    "fa_bwd_check", "fa_bwd", "fa_bwd_stage", "fa_bwd_static", "fa_dropout_mask", "fa_rand",
)

# device scratch of fa_bwd_static (FA_BWD_STATIC_SCRATCH_BYTES in fa_abi.h)
BWD_STATIC_SCRATCH_BYTES = 32 << 20
ERR_SCRATCH = -14

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and type the library; raises FlashAttentionExtensionError."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FlashAttentionExtensionError(
            f"gfx950 kernel library not found at {path}; build it with "
            f"`python flash-attn-v100_amd/build.py`")
    try:
        lib = ctypes.CDLL(path)
    except OSError as e:  # pragma: no cover - depends on the machine
        raise FlashAttentionExtensionError(f"cannot load {path}: {e}") from e
    P = ctypes.POINTER
    lib.fa_abi_version.restype = ctypes.c_int32
    lib.fa_abi_version.argtypes = []
    lib.fa_strerror.restype = ctypes.c_char_p
    lib.fa_strerror.argtypes = [ctypes.c_int32]
    lib.fa_fwd_check.restype = ctypes.c_int32
    lib.fa_fwd_check.argtypes = [P(FwdArgs)]
    lib.fa_fwd.restype = ctypes.c_int32
    lib.fa_fwd.argtypes = [P(FwdArgs), ctypes.c_void_p]
    lib.fa_bwd_workspace_size.restype = ctypes.c_size_t
    lib.fa_bwd_workspace_size.argtypes = [P(BwdArgs)]
    lib.fa_bwd_check.restype = ctypes.c_int32
    lib.fa_bwd_check.argtypes = [P(BwdArgs), ctypes.c_size_t]
    lib.fa_bwd.restype = ctypes.c_int32
    lib.fa_bwd.argtypes = [P(BwdArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.fa_bwd_stage.restype = ctypes.c_int32
    lib.fa_bwd_stage.argtypes = [P(BwdArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_void_p]
    lib.fa_bwd_static.restype = ctypes.c_int32
    lib.fa_bwd_static.argtypes = [P(BwdArgs), ctypes.c_void_p]
    lib.fa_dropout_mask.restype = ctypes.c_int32
    lib.fa_dropout_mask.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int32, ctypes.c_int32,
                                    ctypes.c_int32, ctypes.c_int32, ctypes.c_float, ctypes.c_void_p,
                                    ctypes.c_void_p]
    lib.fa_rand.restype = ctypes.c_int32
    lib.fa_rand.argtypes = [ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    v = lib.fa_abi_version()
    if v != ABI_VERSION:
        raise FlashAttentionExtensionError(f"{path} has ABI version {v}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def strerror(code: int) -> str:
    return load().fa_strerror(code).decode()


def _check(fn: str, code: int) -> None:
    if code != 0:
        raise FlashAttentionKernelError(fn, code, strerror(code))


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def prepare(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` or a copy whose d stride is 1, whose other strides are
    multiples of 16 bytes and whose base is 16-byte aligned (the kernels use
    16-byte vector loads).  Counterpart of the reference's alignment clone
    (kernels/forward_kernel.py:287-300), which re-aligned to 256 bytes."""
    es = t.element_size()
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
          and all(s >= 0 and (s * es) % 16 == 0 for s in t.stride()[:-1]))
    return t if ok else t.clone(memory_format=torch.contiguous_format)


def _strides(t: torch.Tensor):
    return _I64x4(*t.stride())


def padded_head_dim(d: int, dtype: Optional[torch.dtype] = None, bias: bool = False) -> int:
    """The compiled head dim a head dim of ``d`` runs at: the smallest one >= d
    (32, 64, 128; 256 for fp16 / bf16 inputs without a bias, when ``dtype`` is
    given).  Zero columns added to q, k and v change no score (the softmax
    scale is passed explicitly) and make the extra columns of O, dQ, dK and dV
    exactly zero, so the results at d are those of a kernel built for d; the
    dropout stream depends on (b, h, query, key) only, so the mask is the same
    too.  0 for head dims with no kernel."""
    for hd in HEAD_DIMS:
        if 0 < d <= hd:
            return hd
    if d <= WIDE_HEAD_DIM and dtype in (torch.float16, torch.bfloat16) and not bias:
        return WIDE_HEAD_DIM
    return 0


def _pad_d(t: torch.Tensor, dp: int) -> torch.Tensor:
    return t if t.shape[-1] == dp else torch.nn.functional.pad(t, (0, dp - t.shape[-1]))


def _unpad_d(t: torch.Tensor, d: int) -> torch.Tensor:
    return t if t.shape[-1] == d else t[..., :d].contiguous()


def seed_offset(seed: Optional[int], offset: Optional[int]) -> Tuple[int, int]:
    """Dropout Philox seed/offset; undrawn values come from torch's CPU
    generator (no device synchronisation, reproducible under torch.manual_seed)."""
    if seed is None:
        seed = int(torch.randint(0, 2 ** 62, (1,), dtype=torch.int64).item())
    if offset is None:
        offset = 0
    return int(seed) & 0xFFFFFFFFFFFFFFFF, int(offset) & 0xFFFFFFFFFFFFFFFF


class PreparedBias:
    """An additive bias in the layout the kernels read: ``tensor`` viewed as
    (B, H, Sq, Sk) with zero strides on broadcast dimensions, key stride 1,
    other strides multiples of 16 bytes, 16-byte aligned base; element type the
    input dtype or float32.  ``shape`` is the bias's shape as a 4-D view (size 1
    on broadcast dimensions), ``dtype`` its dtype and ``caller_shape`` the shape
    it was given in (2-D, 3-D or 4-D): the gradient is returned in it."""

    __slots__ = ("tensor", "strides", "dtype_code", "shape", "dtype", "caller_shape")

    def __init__(self, tensor, strides, dtype_code, shape, dtype, caller_shape=None):
        self.tensor, self.strides, self.dtype_code, self.shape, self.dtype = tensor, strides, dtype_code, shape, dtype
        self.caller_shape = tuple(shape) if caller_shape is None else tuple(caller_shape)


BIAS_SHAPES_DOC = "[batch|1, heads|1, seq_len_q|1, seq_len_k], [heads, seq_len_q, seq_len_k] or [seq_len_q, seq_len_k]"


def bias_as_4d(bias: torch.Tensor, B: int, H: int, Sq: int, Sk: int) -> torch.Tensor:
    """The bias as a 4-D view: (B|1, H|1, Sq|1, Sk) as it is, (H, Sq, Sk) as
    (1, H, Sq, Sk) and (Sq, Sk) as (1, 1, Sq, Sk) -- the shapes the reference's
    validator accepts (``utils.py:204-211``; its 3-D form is heads-first, "no
    batch dim").  Raises ``ValueError`` for any other shape."""
    if not isinstance(bias, torch.Tensor) or bias.dim() not in (2, 3, 4):
        raise ValueError(f"bias must be a tensor of shape {BIAS_SHAPES_DOC}")
    shape = tuple(bias.shape)
    if bias.dim() == 2:
        if shape != (Sq, Sk):
            raise ValueError(f"bias shape {shape} not compatible with attention shape. Expected {(Sq, Sk)} "
                             f"for a 2-D (position) bias")
        return bias.unsqueeze(0).unsqueeze(0)
    if bias.dim() == 3:
        if shape != (H, Sq, Sk):
            raise ValueError(f"bias shape {shape} not compatible with attention shape. Expected {(H, Sq, Sk)} "
                             f"for a 3-D (per-head) bias")
        return bias.unsqueeze(0)
    want = (B, H, Sq, Sk)
    for d in range(4):
        if shape[d] not in (1, want[d]):
            raise ValueError(f"bias shape {shape} is not broadcastable to {want}")
    return bias


def prepare_bias(bias: torch.Tensor, B: int, H: int, Sq: int, Sk: int, dtype: torch.dtype) -> PreparedBias:
    """Validate a (B|1, H|1, Sq|1, Sk), (H, Sq, Sk) or (Sq, Sk) bias (the
    reference's shapes, utils.py:204-211 and forward_kernel.py:166-182, plus a
    broadcast query dimension) and bring it into the kernels' layout.  A bias
    in the input dtype or float32 is read as it is; any other dtype is converted
    to float32 (exact for float16/bfloat16), so the bias is added in fp32 as the
    reference's Triton kernel did.  Rows are copied into a 16-byte padded
    buffer only when the given strides or base do not meet the kernels'
    alignment."""
    caller_shape = tuple(bias.shape) if isinstance(bias, torch.Tensor) else None
    bias = bias_as_4d(bias, B, H, Sq, Sk)
    shape = tuple(bias.shape)
    orig_dtype = bias.dtype
    t = bias if bias.dtype in (dtype, torch.float32) else bias.to(torch.float32)
    if shape[3] != Sk:  # keys must be contiguous: materialise a broadcast key dimension
        t = t.expand(*shape[:3], Sk)
    es = t.element_size()
    strides = [0 if t.shape[d] == 1 else t.stride(d) for d in range(3)] + [1]
    ok = (t.stride(3) == 1 or Sk <= 1) and t.data_ptr() % 16 == 0 and all(
        s >= 0 and (s * es) % 16 == 0 for s in strides[:3])
    if not ok:
        pad = -(-max(Sk, 1) * es // 16) * 16 // es
        buf = torch.zeros((t.shape[0], t.shape[1], t.shape[2], pad), device=t.device, dtype=t.dtype)
        buf[..., :Sk] = t
        t = buf
        strides = [0 if t.shape[d] == 1 else t.stride(d) for d in range(3)] + [1]
    return PreparedBias(t, _I64x4(*strides), DTYPE_CODES[t.dtype], shape, orig_dtype, caller_shape)


def reduce_dbias(dbias: torch.Tensor, pb: PreparedBias) -> torch.Tensor:
    """Sum the score gradient over the dimensions of the caller's bias that are
    still broadcast (size 1 there, not here), cast it to the bias's dtype and
    give it the caller's shape (a 2-D or 3-D bias gets a 2-D or 3-D gradient)."""
    dims = [d for d in range(4) if pb.shape[d] == 1 and dbias.shape[d] != 1]
    g = dbias.sum(dim=dims, keepdim=True) if dims else dbias
    return g.to(pb.dtype).reshape(pb.caller_shape)


# The dropout keep mask a forward applied, bit-packed: int32 words (B*H*Sq,
# ceil(Sk/32)), bit j%32 of word j/32 of row (b*H + h)*Sq + i.  The autograd
# function keeps it for the backward (one Philox pass instead of three) when it
# takes at most this many bytes.
KEEP_BITS_MAX_BYTES = 4 << 30


def keep_bits_bytes(B: int, H: int, Sq: int, Sk: int) -> int:
    return 4 * B * H * Sq * ((Sk + 31) // 32)


def alloc_keep_bits(B: int, H: int, Sq: int, Sk: int, device) -> torch.Tensor:
    return torch.empty((B * H * Sq, (Sk + 31) // 32), device=device, dtype=torch.int32)


def _check_keep_bits(bits: torch.Tensor, B, H, Sq, Sk, device):
    want = (B * H * Sq, (Sk + 31) // 32)
    if bits.dtype != torch.int32 or tuple(bits.shape) != want or not bits.is_contiguous() or bits.device != device:
        raise ValueError(f"keep bits must be a contiguous int32 {want} tensor on {device}")


def fwd_args(q, k, v, o, lse, max_vals, causal, scale, dropout_p, seed, offset, bias=None,
             keep_bits=None) -> FwdArgs:
    B, Sq, H, D = q.shape
    return FwdArgs(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
        max_vals.data_ptr() if max_vals is not None else None,
        _strides(q), _strides(k), _strides(v), _strides(o),
        B, Sq, k.shape[1], H, k.shape[2], D, DTYPE_CODES[q.dtype], int(bool(causal)),
        float(scale), float(dropout_p), seed, offset,
        bias.tensor.data_ptr() if bias is not None else None,
        bias.strides if bias is not None else _I64x4(0, 0, 0, 1),
        bias.dtype_code if bias is not None else DTYPE_CODES[q.dtype],
        keep_bits.data_ptr() if keep_bits is not None else None)


def _as_prepared(bias, q, k) -> Optional[PreparedBias]:
    if bias is None or isinstance(bias, PreparedBias):
        return bias
    return prepare_bias(bias, q.shape[0], q.shape[2], q.shape[1], k.shape[1], q.dtype)


def fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, scale: float,
        dropout_p: float = 0.0, seed: int = 0, offset: int = 0, want_max: bool = False, bias=None,
        keep_bits: Optional[torch.Tensor] = None):
    """Run ``fa_fwd``: returns (o, lse, max_vals or None).  Inputs (B, S, H, D);
    ``bias`` a (B|1, H|1, Sq|1, Sk), (H, Sq, Sk) or (Sq, Sk) tensor or a
    :class:`PreparedBias`;
    ``keep_bits`` (from :func:`alloc_keep_bits`, with dropout) receives the
    keep mask applied."""
    lib = load()
    D = q.shape[-1]
    dp = padded_head_dim(D, q.dtype, bias is not None) or D  # no kernel: the library rejects it
    q, k, v = (prepare(_pad_d(t, dp)) for t in (q, k, v))
    pb = _as_prepared(bias, q, k)
    B, Sq, H, _ = q.shape
    o = torch.empty_like(q, memory_format=torch.contiguous_format)
    lse = torch.empty((B, H, Sq), device=q.device, dtype=torch.float32)
    mx = torch.empty((B, H, Sq), device=q.device, dtype=torch.float32) if want_max else None
    if keep_bits is not None:
        _check_keep_bits(keep_bits, B, H, Sq, k.shape[1], q.device)
    a = fwd_args(q, k, v, o, lse, mx, causal, scale, dropout_p, seed, offset, pb, keep_bits)
    _check("fa_fwd", lib.fa_fwd(ctypes.byref(a), _stream(q)))
    return _unpad_d(o, D), lse, mx


def bwd_args(q, k, v, o, do, lse, dq, dk, dv, causal, scale, dropout_p, seed, offset,
             bias=None, dbias=None, keep_bits=None) -> BwdArgs:
    B, Sq, H, D = q.shape
    return BwdArgs(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), lse.data_ptr(),
        dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
        _strides(q), _strides(k), _strides(v), _strides(o), _strides(do),
        _strides(dq), _strides(dk), _strides(dv),
        B, Sq, k.shape[1], H, k.shape[2], D, DTYPE_CODES[q.dtype], int(bool(causal)),
        float(scale), float(dropout_p), seed, offset,
        bias.tensor.data_ptr() if bias is not None else None,
        bias.strides if bias is not None else _I64x4(0, 0, 0, 1),
        bias.dtype_code if bias is not None else DTYPE_CODES[q.dtype],
        dbias.data_ptr() if dbias is not None else None,
        _dbias_strides(dbias) if dbias is not None else _I64x4(0, 0, 0, 1),
        DTYPE_CODES[dbias.dtype] if dbias is not None else DTYPE_CODES[torch.float32],
        keep_bits.data_ptr() if keep_bits is not None else None)


def _dbias_strides(dbias):
    # a size-1 batch / head dimension of the gradient buffer asks the library
    # to sum over that dimension (stride 0)
    return _I64x4(*[0 if d < 2 and dbias.shape[d] == 1 else dbias.stride(d) for d in range(4)])


def bwd(q, k, v, o, do, lse, causal: bool, scale: float, dropout_p: float = 0.0,
        seed: int = 0, offset: int = 0, bias=None, want_dbias: bool = False,
        keep_bits: Optional[torch.Tensor] = None):
    """Run ``fa_bwd``: returns (dq, dk, dv) in the input dtype, plus the bias
    gradient in the caller's bias shape and dtype when ``want_dbias``.
    ``keep_bits``: the mask the forward wrote (same seed / offset), read
    instead of regenerating it."""
    lib = load()
    D = q.shape[-1]
    dp = padded_head_dim(D, q.dtype, bias is not None) or D
    q, k, v, o, do = (prepare(_pad_d(t, dp)) for t in (q, k, v, o, do))
    pb = _as_prepared(bias, q, k)
    if want_dbias and pb is None:
        raise ValueError("want_dbias needs a bias")
    lse = lse.contiguous()
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    dbias = None
    if want_dbias:
        B, Sq, H, _ = q.shape
        Sk = k.shape[1]
        # batch / head dimensions the bias broadcasts are summed by the library;
        # every element is written (zeros where causal masks).  A summed
        # gradient's rows are padded to a multiple of 4 keys (the library's rule
        # for its strides).  The library writes the caller's dtype directly unless
        # a query-dimension sum is left to do here (in fp32).
        Bo = 1 if pb.shape[0] == 1 else B
        Ho = 1 if pb.shape[1] == 1 else H
        gdt = pb.dtype if (pb.dtype in DTYPE_CODES and (pb.shape[2] != 1 or Sq == 1)) else torch.float32
        if (Bo, Ho) == (B, H):
            dbias = torch.empty((B, H, Sq, Sk), device=q.device, dtype=gdt)
        else:
            dbias = torch.empty((Bo, Ho, Sq, -(-Sk // 4) * 4), device=q.device, dtype=gdt)[..., :Sk]
    if keep_bits is not None:
        _check_keep_bits(keep_bits, q.shape[0], q.shape[2], q.shape[1], k.shape[1], q.device)
    a = bwd_args(q, k, v, o, do, lse, dq, dk, dv, causal, scale, dropout_p, seed, offset, pb, dbias, keep_bits)
    ws_bytes = lib.fa_bwd_workspace_size(ctypes.byref(a))
    ws = torch.empty(max(int(ws_bytes), 256), device=q.device, dtype=torch.uint8)
    _check("fa_bwd", lib.fa_bwd(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(q)))
    dq, dk, dv = (_unpad_d(t, D) for t in (dq, dk, dv))
    if want_dbias:
        return dq, dk, dv, reduce_dbias(dbias, pb)
    return dq, dk, dv


def bwd_static(q, k, v, o, do, lse, causal: bool, scale: float, dropout_p: float = 0.0,
               seed: int = 0, offset: int = 0, keep_bits: Optional[torch.Tensor] = None):
    """Run ``fa_bwd_static`` (the backward on the library's own device
    scratch, no workspace): returns (dq, dk, dv).  Outputs are allocated here
    by torch; the library call itself allocates nothing."""
    lib = load()
    D = q.shape[-1]
    dp = padded_head_dim(D, q.dtype) or D
    q, k, v, o, do = (prepare(_pad_d(t, dp)) for t in (q, k, v, o, do))
    lse = lse.contiguous()
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    if keep_bits is not None:
        _check_keep_bits(keep_bits, q.shape[0], q.shape[2], q.shape[1], k.shape[1], q.device)
    a = bwd_args(q, k, v, o, do, lse, dq, dk, dv, causal, scale, dropout_p, seed, offset, None, None, keep_bits)
    _check("fa_bwd_static", lib.fa_bwd_static(ctypes.byref(a), _stream(q)))
    return tuple(_unpad_d(t, D) for t in (dq, dk, dv))


def dropout_mask(seed: int, offset: int, B: int, H: int, Sq: int, Sk: int, p: float,
                 device="cuda") -> torch.Tensor:
    """uint8 keep mask (B, H, Sq, Sk) from the kernels' device RNG."""
    lib = load()
    keep = torch.empty((B, H, Sq, Sk), device=device, dtype=torch.uint8)
    _check("fa_dropout_mask", lib.fa_dropout_mask(seed, offset, B, H, Sq, Sk, float(p),
                                                  ctypes.c_void_p(keep.data_ptr()), _stream(keep)))
    return keep


def rand(seed: int, counters: torch.Tensor) -> torch.Tensor:
    """tl.rand(seed, counters) on the device; counters int64/uint64 device tensor."""
    lib = load()
    c = counters.contiguous()
    u = torch.empty(c.shape, device=c.device, dtype=torch.float32)
    _check("fa_rand", lib.fa_rand(seed, ctypes.c_void_p(c.data_ptr()), c.numel(),
                                  ctypes.c_void_p(u.data_ptr()), _stream(c)))
    return u
