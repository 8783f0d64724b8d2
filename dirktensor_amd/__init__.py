"""dirktensor_amd — MI355X (gfx950) HIP implementation of DirkTensor's causal-attention path.

The kernels and the C ABI live in libdirktensor_amd.so (sources in csrc/,
declarations in include/dirktensor_amd.h); this package is the Python mirror
of the reference's FlashAttention.h / OlmoAttention.h interfaces on top of it.
"""

from .attention import (  # noqa: F401
    Context,
    FlashAttentionResult,
    OlmoAttention,
    default_context,
    flash_attention_backward,
    flash_attention_forward,
    qk_norm_rope,
)
from .model import OlmoModel, ce_loss  # noqa: F401
from ._capi import DTError, LIB_PATH  # noqa: F401

__all__ = [
    "Context",
    "DTError",
    "FlashAttentionResult",
    "LIB_PATH",
    "OlmoAttention",
    "OlmoModel",
    "ce_loss",
    "default_context",
    "flash_attention_backward",
    "flash_attention_forward",
    "qk_norm_rope",
]
