"""Autograd layer (reference: ops/__init__.py, ops/attention.py)."""
from .attention import (  # noqa: F401
    EnhancedFlashAttentionV100Function,
    FlashAttentionV100Function,
    SUPPORTED_DTYPES,
)
