"""Autograd wrapper over the gfx950 kernels.

Mirrors ``EnhancedFlashAttentionV100Function`` of mini-kio/flash-attn-v100
(``ops/attention.py:36-333``, alias ``FlashAttentionV100Function`` at ``:756``):
the same 19 leading positional inputs, the same saved-tensor contract
(``save_for_backward`` of the inputs, output and LSE, ``:212``), ``(output, lse)``
when ``return_softmax_lse`` and one gradient slot per input in ``backward``
(``:313-333``).  Two optional trailing inputs carry the dropout Philox seed and
offset so the backward can reproduce the forward's mask (the reference never
saved them, ``:209-227``); with dropout the forward also keeps the mask as bits
for the backward when they fit ``_lib.KEEP_BITS_MAX_BYTES``.

An additive ``bias`` of shape (B|1, H|1, Sq|1, Sk), (H, Sq, Sk) or (Sq, Sk)
(the shapes of the reference's validator, ``utils.py:204-211``) is added to
the scaled scores inside the kernels (reference
``kernels/forward_kernel.py:166-182``) and, when the bias requires grad, its
real gradient dS (summed over broadcast dimensions, in the bias's own shape)
is returned in the bias slot; the reference returned zeros there
(``ops/attention.py:297-301``).

With ``config.DebugConfig.VALIDATE_OUTPUTS`` set, inputs, outputs and
gradients are checked for NaN / Inf as the reference does
(``ops/attention.py:163-168, 203-206, 271-272, 304-310``); off by default.

``enable_gradient_checkpointing`` (or a :func:`gradient_checkpointing_mode`
region) keeps only q, k, v and the LSE: the backward recomputes the output with
one forward pass (deterministic, so the gradients are bit-identical) instead of
holding it between the passes, which saves B*Sq*H*D elements per call.  The
reference recomputed the forward per query segment for dq and ran the full
backward for dk, dv (``ops/attention.py:409-461``), with the same results;
``num_checkpoints`` has no role here and is ignored, and the reference's
automatic switch-on at a 14 GB memory estimate (``:110-124``) is not copied.

Deliberate differences, each raising instead of silently computing something
else: multi-GPU execution is out of scope (``NotImplementedError``);
``block_size_m/n`` are validated hints, the gfx950 tile shape is fixed per
(dtype, head_dim).
"""
from __future__ import annotations

import contextlib
from typing import Any, Dict, Optional, Tuple

import torch

from .. import _lib
from ..config import DebugConfig
from ..utils import check_tensor_nan_inf

SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def check_block_sizes(block_size_m: Optional[int], block_size_n: Optional[int]) -> None:
    """Tile-size hints must be positive multiples of 16 no larger than 256
    (the reference rejects unusable tiles and falls back, tests/test_attention.py:602-625)."""
    for name, val in (("block_size_m", block_size_m), ("block_size_n", block_size_n)):
        if val is None:
            continue
        if not isinstance(val, int) or val <= 0 or val % 16 != 0 or val > 256:
            raise ValueError(f"{name}={val!r} is not a valid tile size (positive multiple of 16, <= 256)")


def _check_kernel_inputs(q, k, v, dropout_p, bias=None):
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("Input tensors must be 4-dimensional [batch, seq_len, num_heads, head_dim]")
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in SUPPORTED_DTYPES:
        raise ValueError(f"dtype must be one of {SUPPORTED_DTYPES} and equal for q, k, v")
    if q.device.type != "cuda" or k.device != q.device or v.device != q.device:
        raise ValueError("Flash Attention requires q, k, v on the same GPU device")
    if not _lib.padded_head_dim(q.shape[-1], q.dtype, bias is not None):
        raise NotImplementedError(
            f"head_dim {q.shape[-1]} has no kernel for {q.dtype}{' with a bias' if bias is not None else ''} "
            f"(1..{_lib.HEAD_DIMS[-1]}, and up to {_lib.WIDE_HEAD_DIM} for fp16 / bf16 without a bias; head dims "
            f"between the compiled {_lib.HEAD_DIMS + (_lib.WIDE_HEAD_DIM,)} run zero-padded to the next one)")
    if k.shape != v.shape or k.shape[0] != q.shape[0] or k.shape[3] != q.shape[3]:
        raise ValueError(f"incompatible shapes q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if k.shape[2] == 0 or q.shape[2] % k.shape[2] != 0:
        raise ValueError(f"num_heads {q.shape[2]} must be a multiple of num_heads_kv {k.shape[2]}")
    if not (0.0 <= dropout_p < 1.0):
        raise ValueError(f"dropout_p must be in [0.0, 1.0), got {dropout_p}")


def _prepare_bias(bias, q, k):
    if bias is None:
        return None
    if not isinstance(bias, torch.Tensor) or bias.device != q.device:
        raise ValueError("bias must be a tensor on the same device as q")
    return _lib.prepare_bias(bias, q.shape[0], q.shape[2], q.shape[1], k.shape[1], q.dtype)


# set by gradient_checkpointing_mode()
_CHECKPOINTING = False


def _keep_bits_for(q, k):
    """A keep-bit buffer for the dropout mask of these inputs, or None past
    ``_lib.KEEP_BITS_MAX_BYTES`` (the backward then regenerates the mask)."""
    B, Sq, H, _ = q.shape
    if _lib.keep_bits_bytes(B, H, Sq, k.shape[1]) > _lib.KEEP_BITS_MAX_BYTES:
        return None
    return _lib.alloc_keep_bits(B, H, Sq, k.shape[1], q.device)


class EnhancedFlashAttentionV100Function(torch.autograd.Function):
    """FlashAttention forward/backward on the gfx950 HIP kernels."""

    @staticmethod
    def forward(
        ctx,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        scale: float,
        causal: bool = False,
        dropout_p: float = 0.0,
        bias: Optional[torch.Tensor] = None,
        block_size_m: Optional[int] = None,
        block_size_n: Optional[int] = None,
        enable_autotuning: bool = True,
        return_softmax_lse: bool = False,
        enable_gradient_checkpointing: bool = False,
        enable_mixed_precision: bool = True,
        num_checkpoints: Optional[int] = None,
        memory_efficient: bool = True,
        performance_mode: str = "balanced",
        enable_multi_gpu: bool = False,
        world_size: int = 1,
        rank: int = 0,
        dropout_seed: Optional[int] = None,
        dropout_offset: Optional[int] = None,
    ):
        if enable_multi_gpu and world_size > 1:
            raise NotImplementedError("multi-GPU execution is out of scope for this single-GPU build")
        check_block_sizes(block_size_m, block_size_n)
        _check_kernel_inputs(q, k, v, dropout_p, bias)
        if scale is None:
            scale = q.shape[-1] ** -0.5
        if DebugConfig.VALIDATE_OUTPUTS:  # reference ops/attention.py:163-168
            for t, name in ((q, "query"), (k, "key"), (v, "value"), (bias, "bias")):
                check_tensor_nan_inf(t, name)
        pb = _prepare_bias(bias, q, k)
        seed, offset = _lib.seed_offset(dropout_seed, dropout_offset) if dropout_p > 0 else (0, 0)
        recompute = bool(enable_gradient_checkpointing) or _CHECKPOINTING
        bits = None
        if dropout_p > 0 and not recompute and any(ctx.needs_input_grad[:3] + ctx.needs_input_grad[6:7]):
            bits = _keep_bits_for(q, k)
        o, lse, _ = _lib.fwd(q, k, v, causal, scale, dropout_p, seed, offset, bias=pb, keep_bits=bits)
        if DebugConfig.VALIDATE_OUTPUTS:  # reference ops/attention.py:203-206 (-inf LSE: a row with no visible key)
            check_tensor_nan_inf(o, "output")
            check_tensor_nan_inf(lse, "lse", allow_neg_inf=True)
        ctx.keep_bits = bits
        ctx.recompute_output = recompute
        kept = (q, k, v, lse) if recompute else (q, k, v, o, lse)
        ctx.save_for_backward(*kept, *(() if pb is None else (pb.tensor,)))
        ctx.bias_meta = None if pb is None else (pb.strides, pb.dtype_code, pb.shape, pb.dtype, pb.caller_shape)
        ctx.scale = scale
        ctx.causal = causal
        ctx.dropout_p = dropout_p
        ctx.seed = seed
        ctx.offset = offset
        ctx.block_size_m = block_size_m
        ctx.block_size_n = block_size_n
        ctx.performance_mode = performance_mode
        if return_softmax_lse:
            ctx.mark_non_differentiable(lse)
            return o, lse
        return o

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor, grad_softmax_lse: Optional[torch.Tensor] = None):
        # grad_softmax_lse is ignored, as in the reference (ops/attention.py:234-333)
        if DebugConfig.VALIDATE_OUTPUTS:  # reference ops/attention.py:271-272
            check_tensor_nan_inf(grad_output, "grad_output")
        saved = ctx.saved_tensors
        n = 4 if ctx.recompute_output else 5
        pb = None if ctx.bias_meta is None else _lib.PreparedBias(saved[n], *ctx.bias_meta)
        bits = ctx.keep_bits
        if ctx.recompute_output:
            # the output again, from the same inputs, seed and offset (same bits);
            # the recomputing pass also records the dropout mask for the backward
            q, k, v, lse = saved[:4]
            if ctx.dropout_p > 0:
                bits = _keep_bits_for(q, k)
            o = _lib.fwd(q, k, v, ctx.causal, ctx.scale, ctx.dropout_p, ctx.seed, ctx.offset,
                         bias=pb, keep_bits=bits)[0]
        else:
            q, k, v, o, lse = saved[:5]
        want_dbias = pb is not None and ctx.needs_input_grad[6]
        grads = _lib.bwd(q, k, v, o, grad_output, lse, ctx.causal, ctx.scale,
                         ctx.dropout_p, ctx.seed, ctx.offset, bias=pb, want_dbias=want_dbias,
                         keep_bits=bits)
        ctx.keep_bits = None
        dq, dk, dv = grads[:3]
        if DebugConfig.VALIDATE_OUTPUTS:  # reference ops/attention.py:304-310
            for t, name in ((dq, "grad_q"), (dk, "grad_k"), (dv, "grad_v"), (grads[3] if want_dbias else None,
                                                                            "grad_bias")):
                check_tensor_nan_inf(t, name)
        return (
            dq if ctx.needs_input_grad[0] else None,
            dk if ctx.needs_input_grad[1] else None,
            dv if ctx.needs_input_grad[2] else None,
            None, None, None,
            grads[3] if want_dbias else None,
            None, None, None, None, None, None,
            None, None, None, None, None, None, None, None,
        )


FlashAttentionV100Function = EnhancedFlashAttentionV100Function


# ---------------------------------------------------------------------------
# Standalone functions (reference ops/attention.py:464-718) and their aliases

def _standalone_inputs(q, k, v, scale, dropout_p, enable_multi_gpu, kwargs, bias=None):
    if enable_multi_gpu and torch.distributed.is_available() and torch.distributed.is_initialized() \
            and torch.distributed.get_world_size() > 1:
        raise NotImplementedError("multi-GPU execution is out of scope for this single-GPU build")
    check_block_sizes(kwargs.get("block_size_m"), kwargs.get("block_size_n"))
    _check_kernel_inputs(q, k, v, dropout_p, bias)
    return q.shape[-1] ** -0.5 if scale is None else scale


def flash_attention_forward_enhanced(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: Optional[float] = None,
    causal: bool = False,
    dropout_p: float = 0.0,
    bias: Optional[torch.Tensor] = None,
    enable_multi_gpu: bool = False,
    performance_mode: str = "balanced",
    **kwargs,
) -> torch.Tensor:
    """Forward only, no autograd graph (reference ``ops/attention.py:464-536``):
    returns O (B, Sq, H, D).  ``dropout_seed`` / ``dropout_offset`` keyword
    arguments pin the dropout stream; ``block_size_m/n`` are validated hints."""
    scale = _standalone_inputs(q, k, v, scale, dropout_p, enable_multi_gpu, kwargs, bias)
    pb = _prepare_bias(bias, q, k)
    seed, offset = (_lib.seed_offset(kwargs.get("dropout_seed"), kwargs.get("dropout_offset"))
                    if dropout_p > 0 else (0, 0))
    with torch.no_grad():
        o, _, _ = _lib.fwd(q, k, v, causal, scale, dropout_p, seed, offset, bias=pb)
    return o


def flash_attention_backward_enhanced(
    grad_output: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    output: torch.Tensor,
    lse: torch.Tensor,
    max_vals: Optional[torch.Tensor],
    scale: float,
    causal: bool = False,
    enable_multi_gpu: bool = False,
    **kwargs,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dQ, dK, dV) from the saved forward state (reference
    ``ops/attention.py:539-600``).  ``lse`` is the LSE this library's forward
    returned; ``max_vals`` is not needed.  A forward that used dropout or a
    bias passes the same ``dropout_p`` / ``dropout_seed`` / ``dropout_offset``
    / ``bias`` as keyword arguments."""
    dropout_p = float(kwargs.get("dropout_p", 0.0))
    scale = _standalone_inputs(q, k, v, scale, dropout_p, enable_multi_gpu, kwargs, kwargs.get("bias"))
    if dropout_p > 0 and kwargs.get("dropout_seed") is None:
        raise ValueError("dropout backward needs the forward's dropout_seed (and dropout_offset)")
    seed, offset = (_lib.seed_offset(kwargs.get("dropout_seed"), kwargs.get("dropout_offset"))
                    if dropout_p > 0 else (0, 0))
    pb = _prepare_bias(kwargs.get("bias"), q, k)
    return _lib.bwd(q, k, v, output, grad_output, lse, causal, scale, dropout_p, seed, offset, bias=pb)


def _reference_attention_fp32(q, k, v, scale, causal, bias, keep, dropout_p):
    """softmax(Q K^T * scale + bias, causal) [* keep / (1 - p)] V in float32 on the
    tensors' device, (B, S, H, D) in and out (the math of reference
    tests/test_attention.py:39-79)."""
    H = q.shape[2]
    rep = H // k.shape[2]
    qf = q.float().transpose(1, 2).contiguous()
    kf = k.float().repeat_interleave(rep, dim=2).transpose(1, 2).contiguous()
    vf = v.float().repeat_interleave(rep, dim=2).transpose(1, 2).contiguous()
    s = torch.matmul(qf, kf.transpose(-2, -1).contiguous()) * scale
    if bias is not None:
        s = s + bias.float()
    if causal:
        m = torch.triu(torch.ones(s.shape[-2], s.shape[-1], device=s.device, dtype=torch.bool), diagonal=1)
        s = s.masked_fill(m, float("-inf"))
    p = torch.softmax(s, dim=-1)
    if keep is not None:
        p = p * keep.float() / (1.0 - dropout_p)
    return torch.matmul(p, vf).transpose(1, 2)


def compare_with_pytorch_attention_enhanced(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    bias: Optional[torch.Tensor] = None,
    dropout_p: float = 0.0,
    atol: float = 1e-4,
    rtol: float = 1e-4,
) -> Dict[str, Any]:
    """The kernels' forward against PyTorch math on the same device, with the
    reference's report keys (``ops/attention.py:603-718``).  The PyTorch side
    runs in float32 (no low-precision batched products) and, for dropout,
    applies the kernels' own keep mask (``fa_dropout_mask``) so that the two
    outputs are comparable element by element; the reference passed dropout
    to SDPA's independent RNG instead."""
    _check_kernel_inputs(q, k, v, dropout_p, bias)
    scale = q.shape[-1] ** -0.5
    seed, offset = _lib.seed_offset(None, None) if dropout_p > 0 else (0, 0)
    flash = flash_attention_forward_enhanced(q, k, v, scale, causal, dropout_p, bias,
                                             dropout_seed=seed, dropout_offset=offset)
    keep = None
    if dropout_p > 0:
        B, Sq, H, _ = q.shape
        keep = _lib.dropout_mask(seed, offset, B, H, Sq, k.shape[1], dropout_p, device=q.device)
    with torch.no_grad():
        ref = _reference_attention_fp32(q, k, v, scale, causal, bias, keep, dropout_p)
    f = flash.float()
    abs_diff = (f - ref).abs()
    rel_diff = abs_diff / (ref.abs() + 1e-8)

    def stats(t):
        return {"mean": t.mean().item(), "std": t.std().item(), "min": t.min().item(), "max": t.max().item()}

    return {
        "allclose": bool(torch.allclose(f, ref, atol=atol, rtol=rtol)),
        "max_absolute_difference": abs_diff.max().item(),
        "mean_absolute_difference": abs_diff.mean().item(),
        "max_relative_difference": rel_diff.max().item(),
        "mean_relative_difference": rel_diff.mean().item(),
        "cosine_similarity": torch.nn.functional.cosine_similarity(f.flatten().unsqueeze(0),
                                                                    ref.flatten().unsqueeze(0)).item(),
        "atol": atol,
        "rtol": rtol,
        "flash_output_stats": stats(f),
        "reference_output_stats": stats(ref),
        "input_shape": q.shape,
        "configuration": {
            "causal": causal,
            "dropout_p": dropout_p,
            "has_bias": bias is not None,
            "dtype": str(q.dtype),
            "device": str(q.device),
        },
    }


@contextlib.contextmanager
def gradient_checkpointing_mode(enable: bool = True):
    """Within the region, attention calls keep only q, k, v and the LSE and
    recompute the output in the backward (as ``enable_gradient_checkpointing``
    does per call).  The reference's context manager is a placeholder
    (``ops/attention.py:721-726``)."""
    global _CHECKPOINTING
    prev = _CHECKPOINTING
    _CHECKPOINTING = bool(enable)
    try:
        yield
    finally:
        _CHECKPOINTING = prev


@contextlib.contextmanager
def mixed_precision_mode(enable: bool = True):
    """Autocast region on the GPU (reference ``ops/attention.py:729-736``)."""
    if enable and torch.cuda.is_available():
        with torch.autocast(device_type="cuda"):
            yield
    else:
        yield


flash_attention_forward = flash_attention_forward_enhanced
flash_attention_backward = flash_attention_backward_enhanced
compare_with_pytorch_attention = compare_with_pytorch_attention_enhanced
