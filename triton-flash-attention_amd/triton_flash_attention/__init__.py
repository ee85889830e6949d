"""MI355X-native FlashAttention-2 with the public API of triton_flash_attention.

Same import surface as the reference package (triton_flash_attention/__init__.py:3-15).
"""

from .attention import (
    DispatchDecision,
    TritonAttention,
    explain_dispatch,
    scaled_dot_product_attention,
)

__version__ = "0.2.0+gfx950"

__all__ = [
    "DispatchDecision",
    "TritonAttention",
    "explain_dispatch",
    "scaled_dot_product_attention",
]
