"""Forward launchers with the reference's names and signatures.

``flash_attention_forward_triton_enhanced`` (reference
``kernels/forward_kernel.py:246-387``) and
``flash_attention_forward_autotuned_enhanced`` (``:445-512``) both return
``(o, lse, max_vals)``: ``o`` in the input dtype, ``lse`` and ``max_vals``
(B, H, Sq) float32.  Here ``lse`` is the natural-log logsumexp of the scaled,
biased, masked scores (the reference stored the row sum under that name) and
``max_vals`` the row max of the scaled, biased scores.  ``bias`` is an additive
(B|1, H|1, Sq|1, Sk) tensor added in fp32 after the scale and before the causal
mask, as at ``kernels/forward_kernel.py:166-182``.  The Triton-tuning switches
(warp specialisation, double buffering, prefetch, fast math) are accepted and
have no effect: the gfx950 kernel always double-buffers K/V and uses exp2.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import _lib
from ..ops.attention import _check_kernel_inputs, _prepare_bias, check_block_sizes


def flash_attention_forward_triton_enhanced(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    causal: bool = False,
    dropout_p: float = 0.0,
    bias: Optional[torch.Tensor] = None,
    block_size_m: int = 64,
    block_size_n: int = 64,
    enable_warp_specialization: bool = True,
    enable_double_buffering: bool = True,
    enable_prefetch: bool = True,
    use_fast_math: bool = False,
    dropout_seed: Optional[int] = None,
    dropout_offset: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    check_block_sizes(block_size_m, block_size_n)
    _check_kernel_inputs(q, k, v, dropout_p)
    pb = _prepare_bias(bias, q, k)
    seed, offset = _lib.seed_offset(dropout_seed, dropout_offset) if dropout_p > 0 else (0, 0)
    return _lib.fwd(q, k, v, causal, scale, dropout_p, seed, offset, want_max=True, bias=pb)


def flash_attention_forward_autotuned_enhanced(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    causal: bool = False,
    dropout_p: float = 0.0,
    bias: Optional[torch.Tensor] = None,
    dropout_seed: Optional[int] = None,
    dropout_offset: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The reference's default path (its kernel body was ``pass``); here the
    same static gfx950 kernel as the non-autotuned launcher."""
    return flash_attention_forward_triton_enhanced(
        q, k, v, scale, causal, dropout_p, bias, None, None,
        dropout_seed=dropout_seed, dropout_offset=dropout_offset)
