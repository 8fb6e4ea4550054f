"""Backward launcher with the reference's name and signature
(``kernels/backward_kernel.py:208-318``): returns ``(dq, dk, dv)`` in the input
dtype.  ``lse`` must be the LSE written by the forward of this library;
``max_vals`` is accepted for signature compatibility and not needed.  Dropout
is honoured when ``dropout_p``/``dropout_seed``/``dropout_offset`` match the
forward call (the reference's backward ignored dropout).  A forward that used
an additive ``bias`` needs the same ``bias`` here; ``return_dbias=True`` then
appends its gradient (the bias's shape and dtype) as a fourth element."""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import _lib
from ..ops.attention import _check_kernel_inputs, _prepare_bias, check_block_sizes


def flash_attention_backward_triton_enhanced(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    do: torch.Tensor,
    lse: torch.Tensor,
    max_vals: Optional[torch.Tensor],
    scale: float,
    causal: bool = False,
    block_size_m: int = 64,
    block_size_n: int = 64,
    enable_fused_delta: bool = True,
    enable_gradient_accumulation: bool = True,
    use_fast_math: bool = False,
    dropout_p: float = 0.0,
    dropout_seed: Optional[int] = None,
    dropout_offset: Optional[int] = None,
    bias: Optional[torch.Tensor] = None,
    return_dbias: bool = False,
) -> Tuple[torch.Tensor, ...]:
    check_block_sizes(block_size_m, block_size_n)
    _check_kernel_inputs(q, k, v, dropout_p)
    if dropout_p > 0 and dropout_seed is None:
        raise ValueError("dropout backward needs the forward's dropout_seed (and dropout_offset)")
    pb = _prepare_bias(bias, q, k)
    seed, offset = _lib.seed_offset(dropout_seed, dropout_offset) if dropout_p > 0 else (0, 0)
    return _lib.bwd(q, k, v, o, do, lse, causal, scale, dropout_p, seed, offset,
                    bias=pb, want_dbias=return_dbias)
