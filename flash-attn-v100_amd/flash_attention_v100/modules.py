"""Multi-head attention layer over the gfx950 kernels.

``EnhancedMultiHeadAttention`` keeps the constructor and ``forward`` of the
reference's module (``examples/basic_usage.py:48-255``): Q/K/V/output linear
projections with Xavier-uniform weights and zero biases, (B, S, E) or
(S, B, E) inputs, boolean ``attn_mask`` / ``key_padding_mask`` turned into an
additive ``-inf`` bias, ``is_causal``, dropout only in training mode, and an
``(output, attn_weights)`` return whose weights are not computed.

Differences, all deliberate:

* The masks become a bias that broadcasts over the dimensions they do not
  name ((1|B, 1, Sq|1, Sk)) instead of a materialised (B, H, Sq, Sk) tensor;
  the kernels read broadcast dimensions with stride 0.  A float ``attn_mask``
  is added as it is (the reference's ``masked_fill`` accepted booleans only).
* A query row whose keys are all masked gives zeros (the reference's softmax
  gave NaN there).
* ``enable_gradient_checkpointing`` is honoured: the layer's attention keeps
  only q, k, v and the LSE for the backward (the reference stored the flag).
* ``enable_performance_monitoring`` times each forward with HIP events on the
  current stream (the reference used its profiler module, which is out of
  scope); :meth:`get_performance_stats` reports count and mean milliseconds.
* ``enable_multi_gpu`` is accepted and ignored (one GPU).
"""
from __future__ import annotations

import contextlib
import warnings
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn

from .interface import flash_attention_performance_mode, flash_attention_v100
from .ops.attention import gradient_checkpointing_mode


def mask_to_bias(attn_mask: Optional[torch.Tensor], key_padding_mask: Optional[torch.Tensor], batch: int,
                 seq_q: int, seq_k: int, dtype: torch.dtype, device) -> Optional[torch.Tensor]:
    """Additive bias of shape (1|B, 1, Sq|1, Sk) from the reference's masks
    (``examples/basic_usage.py:232-251``): a True entry of a boolean mask
    removes that key (-inf); a float ``attn_mask`` is added as it is.
    ``attn_mask`` is (Sq, Sk) or (B, Sq, Sk); ``key_padding_mask`` is (B, Sk)."""
    if attn_mask is None and key_padding_mask is None:
        return None
    bias = None
    if attn_mask is not None:
        if attn_mask.dim() not in (2, 3):
            raise ValueError(f"attn_mask must be 2-D (Sq, Sk) or 3-D (B, Sq, Sk), got shape {tuple(attn_mask.shape)}")
        am = attn_mask.to(device)
        if am.dtype == torch.bool:
            am = torch.zeros(am.shape, device=device, dtype=dtype).masked_fill(am, float("-inf"))
        else:
            am = am.to(dtype)
        bias = am.unsqueeze(0).unsqueeze(0) if am.dim() == 2 else am.unsqueeze(1)
        if bias.shape[-2:] != (seq_q, seq_k) or bias.shape[0] not in (1, batch):
            raise ValueError(f"attn_mask shape {tuple(attn_mask.shape)} does not match (B={batch}, Sq={seq_q}, "
                             f"Sk={seq_k})")
    if key_padding_mask is not None:
        if tuple(key_padding_mask.shape) != (batch, seq_k):
            raise ValueError(f"key_padding_mask must be (B={batch}, Sk={seq_k}), got {tuple(key_padding_mask.shape)}")
        kp = key_padding_mask.to(device)
        if kp.dtype == torch.bool:
            kp = torch.zeros(kp.shape, device=device, dtype=dtype).masked_fill(kp, float("-inf"))
        else:
            kp = kp.to(dtype)
        kp = kp.view(batch, 1, 1, seq_k)
        bias = kp if bias is None else bias + kp
    return bias


class EnhancedMultiHeadAttention(nn.Module):
    """Multi-head attention with the reference's module interface
    (``examples/basic_usage.py:48-255``) over :func:`flash_attention_v100`."""

    def __init__(self,
                 embed_dim: int,
                 num_heads: int,
                 dropout: float = 0.0,
                 bias: bool = True,
                 batch_first: bool = True,
                 optimization_strategy: str = "balanced",
                 enable_multi_gpu: bool = True,
                 enable_gradient_checkpointing: bool = False,
                 enable_performance_monitoring: bool = False):
        super().__init__()
        assert embed_dim % num_heads == 0, "embed_dim must be divisible by num_heads"
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.head_dim = embed_dim // num_heads
        self.dropout = dropout
        self.batch_first = batch_first
        self.optimization_strategy = optimization_strategy
        self.enable_multi_gpu = enable_multi_gpu
        self.enable_gradient_checkpointing = enable_gradient_checkpointing
        self.enable_performance_monitoring = enable_performance_monitoring
        self.q_proj = nn.Linear(embed_dim, embed_dim, bias=bias)
        self.k_proj = nn.Linear(embed_dim, embed_dim, bias=bias)
        self.v_proj = nn.Linear(embed_dim, embed_dim, bias=bias)
        self.out_proj = nn.Linear(embed_dim, embed_dim, bias=bias)
        self.forward_count = 0
        self._times_ms = []
        self._pending = []
        self.reset_parameters()

    def reset_parameters(self):
        """Xavier-uniform projection weights, zero biases (reference ``:112-123``)."""
        for lin in (self.q_proj, self.k_proj, self.v_proj, self.out_proj):
            nn.init.xavier_uniform_(lin.weight)
            if lin.bias is not None:
                nn.init.constant_(lin.bias, 0)

    def forward(self,
                query: torch.Tensor,
                key: Optional[torch.Tensor] = None,
                value: Optional[torch.Tensor] = None,
                key_padding_mask: Optional[torch.Tensor] = None,
                attn_mask: Optional[torch.Tensor] = None,
                need_weights: bool = False,
                average_attn_weights: bool = True,
                is_causal: bool = False) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """(output, attn_weights); see the module docstring.  ``need_weights``
        warns and returns zeros of shape (B, H, Sq, Sk), as the reference does
        (``:194-199, 218-221``): the kernels never form the weights."""
        timing = self.enable_performance_monitoring and query.is_cuda
        if timing:
            self.forward_count += 1
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record()
        if not self.batch_first:
            query = query.transpose(0, 1)
            key = key.transpose(0, 1) if key is not None else None
            value = value.transpose(0, 1) if value is not None else None
        if key is None:
            key = query
        if value is None:
            value = key
        B, Sq, E = query.shape
        Sk = key.shape[1]
        q = self.q_proj(query).view(B, Sq, self.num_heads, self.head_dim)
        k = self.k_proj(key).view(B, Sk, self.num_heads, self.head_dim)
        v = self.v_proj(value).view(B, value.shape[1], self.num_heads, self.head_dim)
        bias = mask_to_bias(attn_mask, key_padding_mask, B, Sq, Sk, q.dtype, q.device)
        if need_weights:
            warnings.warn("need_weights=True not supported with Flash Attention. "
                          "Attention weights will not be returned.", UserWarning)
        ckpt = gradient_checkpointing_mode() if self.enable_gradient_checkpointing else contextlib.nullcontext()
        with flash_attention_performance_mode(self.optimization_strategy), ckpt:
            out = flash_attention_v100(q, k, v, causal=is_causal,
                                       dropout_p=self.dropout if self.training else 0.0,
                                       bias=bias, optimization_strategy=self.optimization_strategy,
                                       enable_multi_gpu=self.enable_multi_gpu,
                                       enable_profiling=self.enable_performance_monitoring,
                                       fallback_on_error=True)
        out = self.out_proj(out.reshape(B, Sq, E))
        if not self.batch_first:
            out = out.transpose(0, 1)
        weights = None
        if need_weights:
            weights = torch.zeros(B, self.num_heads, Sq, Sk, device=out.device, dtype=out.dtype)
        if timing:
            ev1.record()
            self._pending.append((ev0, ev1))
        return out, weights

    def get_performance_stats(self) -> Optional[Dict[str, Any]]:
        """Forward count and HIP-event times (ms) when monitoring is enabled."""
        if not self.enable_performance_monitoring:
            return None
        for ev0, ev1 in self._pending:
            ev1.synchronize()
            self._times_ms.append(ev0.elapsed_time(ev1))
        self._pending = []
        n = len(self._times_ms)
        return {"forward_count": self.forward_count,
                "mean_ms": sum(self._times_ms) / n if n else None,
                "total_ms": sum(self._times_ms)}
