"""Autograd layer and standalone functions (reference: ops/__init__.py,
ops/attention.py).  The reference's memory pool (ops/memory.py) is not part of
this build: torch's caching allocator owns all memory."""
from .attention import (  # noqa: F401
    EnhancedFlashAttentionV100Function,
    FlashAttentionV100Function,
    SUPPORTED_DTYPES,
    compare_with_pytorch_attention,
    compare_with_pytorch_attention_enhanced,
    flash_attention_backward,
    flash_attention_backward_enhanced,
    flash_attention_forward,
    flash_attention_forward_enhanced,
    gradient_checkpointing_mode,
    mixed_precision_mode,
)

__all__ = [
    "FlashAttentionV100Function",
    "EnhancedFlashAttentionV100Function",
    "flash_attention_forward",
    "flash_attention_backward",
    "compare_with_pytorch_attention",
    "flash_attention_forward_enhanced",
    "flash_attention_backward_enhanced",
    "compare_with_pytorch_attention_enhanced",
    "gradient_checkpointing_mode",
    "mixed_precision_mode",
]
