"""Public entry point with the reference's signature (``interface.py:199-349``).

``flash_attention_v100(q, k, v, causal, scale, dropout_p, bias, block_size_m,
block_size_n, enable_autotuning, return_softmax_lse, optimization_strategy,
enable_multi_gpu, enable_profiling, fallback_on_error, validate_inputs)`` on
(B, S, H, D) tensors returns O (B, Sq, H, D) in q's dtype, or ``(O, LSE)``.

Single GPU only: the reference's Manager and its multi-GPU dispatch
(``interface.py:25-196, 351-450``) are out of scope.  Validation checks
metadata only by default (no full-tensor scans, no host synchronisation; the
reference's ``utils.py:219-254`` scans cost a sync each); setting
``config.DebugConfig.CHECK_NUMERICAL_STABILITY`` turns those scans on.  A bias
may be (B|1, H|1, Sq|1, Sk), (H, Sq, Sk) or (Sq, Sk) (reference
``utils.py:204-211``).

Fallback (reference ``interface.py:331-348, 453-490``): with
``fallback_on_error=True`` a request the gfx950 kernels do not implement
(``NotImplementedError``: a head_dim above 256, or above 128 for float32
inputs or with a bias; others between the compiled 32 / 64 / 128 / 256 run
zero-padded to the next) or reject as a
tile hint (``ValueError`` from ``block_size_m/n``) is served by PyTorch math on
the same GPU, with a warning.  Everything else raises: a missing kernel library
(:class:`FlashAttentionExtensionError`), a kernel error, CPU tensors (there is
no CPU path).
"""
from __future__ import annotations

import contextlib
import math
import warnings
from typing import Optional, Tuple, Union

import torch

from . import _lib
from .config import DebugConfig
from .utils import check_numerical_stability
from .ops.attention import FlashAttentionV100Function, SUPPORTED_DTYPES, check_block_sizes

_STRATEGIES = ("speed", "memory", "balanced", "adaptive")


class _Stats:
    """Counter of fallbacks taken (reference: Manager.error_recovery_count)."""
    error_recovery_count = 0


def validate_inputs_enhanced(q, k, v, scale=None, bias=None, dropout_p=0.0):
    """Metadata checks with the reference's error types and messages
    (``utils.py:31-160``); returns (q, k, v, scale) with the default
    ``scale = head_dim ** -0.5`` (``utils.py:148-153``)."""
    if not all(isinstance(t, torch.Tensor) for t in (q, k, v)):
        raise TypeError("q, k, v must be torch.Tensor instances")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("Input tensors must be 4-dimensional [batch, seq_len, num_heads, head_dim]")
    B, Sq, Hq, Dq = q.shape
    Bk, Sk, Hk, Dk = k.shape
    Bv, Sv, Hv, Dv = v.shape
    if not (B == Bk == Bv):
        raise ValueError(f"Batch sizes must match across Q, K, V. Got Q: {B}, K: {Bk}, V: {Bv}")
    if Sk != Sv:
        raise ValueError(f"Sequence lengths of K and V must match. Got K: {Sk}, V: {Sv}")
    if not (Dq == Dk == Dv):
        raise ValueError(f"Head dimensions must match across Q, K, V. Got Q: {Dq}, K: {Dk}, V: {Dv}")
    if Hk == 0 or Hv == 0 or Hq % Hk != 0 or Hq % Hv != 0:
        raise ValueError(f"Number of query heads ({Hq}) must be divisible by number of key heads ({Hk}) "
                         f"and value heads ({Hv})")
    if Hk != Hv:
        raise ValueError(f"Number of key heads ({Hk}) must equal number of value heads ({Hv})")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"All tensors must have the same dtype. Got Q: {q.dtype}, K: {k.dtype}, V: {v.dtype}")
    if q.dtype not in SUPPORTED_DTYPES:
        raise ValueError(f"Unsupported dtype {q.dtype}. Supported types: "
                         + ", ".join(str(d) for d in SUPPORTED_DTYPES))
    if not (q.device == k.device == v.device):
        raise ValueError(f"All tensors must be on the same device. Got Q: {q.device}, K: {k.device}, V: {v.device}")
    if q.device.type != "cuda":
        raise ValueError("Flash Attention requires GPU tensors (there is no CPU path)")
    if bias is not None:
        if not isinstance(bias, torch.Tensor):
            raise TypeError("bias must be a torch.Tensor")
        _lib.bias_as_4d(bias, B, Hq, Sq, Sk)  # the reference's shapes (utils.py:204-211), ValueError else
        if bias.device != q.device:
            raise ValueError(f"bias must be on {q.device}, got {bias.device}")
    if not (0.0 <= dropout_p < 1.0):
        raise ValueError(f"dropout_p must be in [0.0, 1.0), got {dropout_p}")
    if scale is None:
        scale = Dq ** -0.5
    if not (math.isfinite(scale) and scale > 0):
        raise ValueError(f"scale must be finite and positive, got {scale}")
    if DebugConfig.CHECK_NUMERICAL_STABILITY:  # reference utils.py:142, 219-254 (opt-in here)
        check_numerical_stability(q, k, v, bias)
    return q, k, v, scale


def _fallback_to_pytorch(q, k, v, scale, causal, dropout_p, bias, return_softmax_lse, dropout_seed=None,
                         dropout_offset=None):
    """PyTorch math on the tensors' GPU, computed in float32 (reference
    ``interface.py:453-490`` used SDPA).  Returns a real LSE, unlike the
    reference's zeros.  Dropout applies the kernels' Philox mask for the same
    seed and offset (drawn by the library's mask kernel), so a seed means the
    same mask on both paths."""
    if q.device.type != "cuda":
        raise ValueError("fallback requires GPU tensors")
    H = q.shape[2]
    rep = H // k.shape[2]
    qf = q.float().transpose(1, 2)
    kf = k.float().repeat_interleave(rep, dim=2).transpose(1, 2).contiguous()
    vf = v.float().repeat_interleave(rep, dim=2).transpose(1, 2).contiguous()
    s = torch.matmul(qf, kf.transpose(-2, -1).contiguous()) * scale
    if bias is not None:
        s = s + bias.float()
    if causal:
        mask = torch.triu(torch.ones(s.shape[-2], s.shape[-1], device=s.device, dtype=torch.bool), diagonal=1)
        s = s.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.softmax(s, dim=-1)
    if dropout_p > 0:
        seed, offset = _lib.seed_offset(dropout_seed, dropout_offset)
        keep = _lib.dropout_mask(seed, offset, s.shape[0], s.shape[1], s.shape[2], s.shape[3], dropout_p, q.device)
        p = p * keep.to(p.dtype) / (1.0 - dropout_p)
    o = torch.matmul(p, vf).transpose(1, 2).to(q.dtype)
    return (o, lse) if return_softmax_lse else o


def flash_attention_v100(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    scale: Optional[float] = None,
    dropout_p: float = 0.0,
    bias: Optional[torch.Tensor] = None,
    block_size_m: Optional[int] = None,
    block_size_n: Optional[int] = None,
    enable_autotuning: bool = True,
    return_softmax_lse: bool = False,
    optimization_strategy: str = "balanced",
    enable_multi_gpu: Optional[bool] = None,
    enable_profiling: bool = False,
    fallback_on_error: bool = True,
    validate_inputs: bool = True,
    *,
    dropout_seed: Optional[int] = None,
    dropout_offset: Optional[int] = None,
) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """FlashAttention on (B, S, H, D) tensors; see the module docstring.

    ``optimization_strategy`` (speed / memory / balanced / adaptive) selects
    among numerically identical configurations and is validated only;
    ``enable_multi_gpu`` and ``enable_profiling`` are accepted for signature
    compatibility (single GPU; profile with rocprofv3).  ``dropout_seed`` /
    ``dropout_offset`` pin the Philox stream of the dropout mask (drawn from
    torch's CPU generator when omitted).
    """
    if optimization_strategy not in _STRATEGIES:
        raise ValueError(f"optimization_strategy must be one of {_STRATEGIES}, got {optimization_strategy!r}")
    if validate_inputs:
        q, k, v, scale = validate_inputs_enhanced(q, k, v, scale, bias, dropout_p)
    elif scale is None:
        scale = q.shape[-1] ** -0.5
    try:
        check_block_sizes(block_size_m, block_size_n)
        return FlashAttentionV100Function.apply(
            q, k, v, scale, causal, dropout_p, bias, block_size_m, block_size_n,
            enable_autotuning, return_softmax_lse, False, True, None, True,
            optimization_strategy, False, 1, 0, dropout_seed, dropout_offset)
    except (NotImplementedError, ValueError) as e:
        if isinstance(e, _lib.FlashAttentionExtensionError) or not fallback_on_error:
            raise
        warnings.warn(f"Flash Attention failed ({e}), falling back to PyTorch implementation", UserWarning)
        _Stats.error_recovery_count += 1
        return _fallback_to_pytorch(q, k, v, scale, causal, dropout_p, bias, return_softmax_lse, dropout_seed,
                                    dropout_offset)


# Convenience entry points and context managers of the reference
# (interface.py:611-669).  The strategies select among numerically identical
# kernel configurations here, so a performance mode only records the strategy.

def flash_attention_v100_causal(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, **kwargs) -> torch.Tensor:
    """Causal attention (reference ``interface.py:611-618``)."""
    return flash_attention_v100(q, k, v, causal=True, **kwargs)


def flash_attention_v100_with_dropout(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dropout_p: float,
                                      **kwargs) -> torch.Tensor:
    """Attention with dropout (reference ``interface.py:621-629``)."""
    return flash_attention_v100(q, k, v, dropout_p=dropout_p, **kwargs)


_current_strategy = ["balanced"]


def current_optimization_strategy() -> str:
    """The strategy set by the innermost :func:`flash_attention_performance_mode`."""
    return _current_strategy[-1]


@contextlib.contextmanager
def flash_attention_performance_mode(strategy: str = "speed"):
    """Run a region under an optimization strategy (reference
    ``interface.py:644-654``, which swapped its global Manager).  The strategy is
    validated and exposed through :func:`current_optimization_strategy`."""
    if strategy not in _STRATEGIES:
        raise ValueError(f"optimization_strategy must be one of {_STRATEGIES}, got {strategy!r}")
    _current_strategy.append(strategy)
    try:
        yield
    finally:
        _current_strategy.pop()


@contextlib.contextmanager
def flash_attention_memory_mode():
    """``flash_attention_performance_mode('memory')`` (reference ``interface.py:657-661``)."""
    with flash_attention_performance_mode("memory"):
        yield
