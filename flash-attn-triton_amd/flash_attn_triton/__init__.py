"""FlashAttention-2 forward for AMD MI355X (gfx950), with the API of flash_attn_triton.

Drop-in for luyanaa/flash-attn-triton's import surface
(``flash_attn_triton/__init__.py:6-18`` of the reference).  The kernels are
hand-written HIP for CDNA4 in ``libfa_gfx950.so``; there is no Triton inside
despite the package name, which is kept so existing imports resolve.
"""

__version__ = "0.1.1+gfx950"

from .flash_attn_interface import (
    flash_attn_func,
    flash_attn_func_cross,
    flash_attn_qkvpacked_func,
    flash_attn_kvpacked_func,
    flash_attn_with_kvcache,
    FlashAttention,
    flash_attn_varlen_func,
    flash_attn_varlen_qkvpacked_func,
    flash_attn_varlen_kvpacked_func,
    FlashSelfAttention,
    FlashCrossAttention,
)
