"""Kernel-level entry points (reference: kernels/__init__.py, forward_kernel.py,
backward_kernel.py): the launchers FlashAttentionV100Function calls, now
backed by the gfx950 HIP library instead of Triton."""
from .backward_kernel import flash_attention_backward_triton_enhanced  # noqa: F401
from .forward_kernel import (  # noqa: F401
    flash_attention_forward_autotuned_enhanced,
    flash_attention_forward_triton_enhanced,
)
