"""FlashAttention forward/backward for AMD Instinct MI355X (gfx950).

Drop-in for the public surface of mini-kio/flash-attn-v100's hot path:
``flash_attention_v100`` (reference ``interface.py:199``),
``FlashAttentionV100Function`` (``ops/attention.py:36, 756``) and the kernel
launchers (``kernels/forward_kernel.py:246, 445``,
``kernels/backward_kernel.py:208``), all backed by hand-written HIP kernels in
``libfa_gfx950.so`` (C ABI: ``include/fa_abi.h``).  Importing the package does
not load the library; the first kernel call does, and raises
``FlashAttentionExtensionError`` if it is missing.
"""
from ._lib import FlashAttentionExtensionError, FlashAttentionKernelError  # noqa: F401
from .interface import (  # noqa: F401
    flash_attention_memory_mode,
    flash_attention_performance_mode,
    flash_attention_v100,
    flash_attention_v100_causal,
    flash_attention_v100_with_dropout,
    validate_inputs_enhanced,
)
from .kernels import (  # noqa: F401
    flash_attention_backward_triton_enhanced,
    flash_attention_forward_autotuned_enhanced,
    flash_attention_forward_triton_enhanced,
)
from .ops.attention import (  # noqa: F401
    EnhancedFlashAttentionV100Function,
    FlashAttentionV100Function,
    SUPPORTED_DTYPES,
    compare_with_pytorch_attention,
    flash_attention_backward,
    flash_attention_forward,
)
from .modules import EnhancedMultiHeadAttention  # noqa: F401
from .config import DebugConfig  # noqa: F401
from .utils import check_tensor_nan_inf  # noqa: F401

__version__ = "0.1.0"

__all__ = [
    "flash_attention_v100",
    "flash_attention_v100_causal",
    "flash_attention_v100_with_dropout",
    "flash_attention_performance_mode",
    "flash_attention_memory_mode",
    "EnhancedMultiHeadAttention",
    "FlashAttentionV100Function",
    "EnhancedFlashAttentionV100Function",
    "flash_attention_forward_triton_enhanced",
    "flash_attention_forward_autotuned_enhanced",
    "flash_attention_backward_triton_enhanced",
    "validate_inputs_enhanced",
    "FlashAttentionExtensionError",
    "FlashAttentionKernelError",
    "SUPPORTED_DTYPES",
    "flash_attention_forward",
    "flash_attention_backward",
    "compare_with_pytorch_attention",
    "DebugConfig",
    "check_tensor_nan_inf",
]
