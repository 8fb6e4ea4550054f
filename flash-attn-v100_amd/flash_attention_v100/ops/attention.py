"""Autograd wrapper over the gfx950 kernels.

Mirrors ``EnhancedFlashAttentionV100Function`` of mini-kio/flash-attn-v100
(``ops/attention.py:36-333``, alias ``FlashAttentionV100Function`` at ``:756``):
the same 19 leading positional inputs, the same saved-tensor contract
(``save_for_backward`` of the inputs, output and LSE, ``:212``), ``(output, lse)``
when ``return_softmax_lse`` and one gradient slot per input in ``backward``
(``:313-333``).  Two optional trailing inputs carry the dropout Philox seed and
offset so the backward regenerates the forward's mask (the reference never saved
them, ``:209-227``).

An additive ``bias`` of shape (B|1, H|1, Sq|1, Sk) is added to the scaled
scores inside the kernels (reference ``kernels/forward_kernel.py:166-182``)
and, when the bias requires grad, its real gradient dS (summed over broadcast
dimensions) is returned in the bias slot; the reference returned zeros there
(``ops/attention.py:297-301``).

Deliberate differences, each raising instead of silently computing something
else: multi-GPU execution is out of scope (``NotImplementedError``);
``enable_gradient_checkpointing`` is accepted and has nothing to do (the
backward already recomputes P tile by tile); ``block_size_m/n`` are validated
hints, the gfx950 tile shape is fixed per (dtype, head_dim).
"""
from __future__ import annotations

from typing import Optional

import torch

from .. import _lib

SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def check_block_sizes(block_size_m: Optional[int], block_size_n: Optional[int]) -> None:
    """Tile-size hints must be positive multiples of 16 no larger than 256
    (the reference rejects unusable tiles and falls back, tests/test_attention.py:602-625)."""
    for name, val in (("block_size_m", block_size_m), ("block_size_n", block_size_n)):
        if val is None:
            continue
        if not isinstance(val, int) or val <= 0 or val % 16 != 0 or val > 256:
            raise ValueError(f"{name}={val!r} is not a valid tile size (positive multiple of 16, <= 256)")


def _check_kernel_inputs(q, k, v, dropout_p):
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("Input tensors must be 4-dimensional [batch, seq_len, num_heads, head_dim]")
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in SUPPORTED_DTYPES:
        raise ValueError(f"dtype must be one of {SUPPORTED_DTYPES} and equal for q, k, v")
    if q.device.type != "cuda" or k.device != q.device or v.device != q.device:
        raise ValueError("Flash Attention requires q, k, v on the same GPU device")
    if q.shape[-1] not in _lib.HEAD_DIMS:
        raise NotImplementedError(f"head_dim {q.shape[-1]} is not compiled (supported: {_lib.HEAD_DIMS})")
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
        _check_kernel_inputs(q, k, v, dropout_p)
        if scale is None:
            scale = q.shape[-1] ** -0.5
        pb = _prepare_bias(bias, q, k)
        seed, offset = _lib.seed_offset(dropout_seed, dropout_offset) if dropout_p > 0 else (0, 0)
        o, lse, _ = _lib.fwd(q, k, v, causal, scale, dropout_p, seed, offset, bias=pb)
        if pb is None:
            ctx.save_for_backward(q, k, v, o, lse)
        else:
            ctx.save_for_backward(q, k, v, o, lse, pb.tensor)
        ctx.bias_meta = None if pb is None else (pb.strides, pb.dtype_code, pb.shape, pb.dtype)
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
        saved = ctx.saved_tensors
        q, k, v, o, lse = saved[:5]
        pb = None if ctx.bias_meta is None else _lib.PreparedBias(saved[5], *ctx.bias_meta)
        want_dbias = pb is not None and ctx.needs_input_grad[6]
        grads = _lib.bwd(q, k, v, o, grad_output, lse, ctx.causal, ctx.scale,
                         ctx.dropout_p, ctx.seed, ctx.offset, bias=pb, want_dbias=want_dbias)
        dq, dk, dv = grads[:3]
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
