"""FlashAttention-2 compatibility facade (reference ``flash_attn/__init__.py:1-22``).

Lets ``from flash_attn import flash_attn_func`` resolve to the gfx950 build.
"""

from flash_attn_triton.flash_attn_interface import (
    flash_attn_func,
    flash_attn_qkvpacked_func,
    flash_attn_kvpacked_func,
    flash_attn_with_kvcache,
    FlashAttention,
    flash_attn_varlen_func,
    flash_attn_varlen_qkvpacked_func,
    flash_attn_varlen_kvpacked_func,
)

# FlashAttention 1.x names (renamed in FA2).
from flash_attn_triton.flash_attn_interface import (
    flash_attn_varlen_func as flash_attn_unpadded_func,
    flash_attn_varlen_qkvpacked_func as flash_attn_unpadded_qkvpacked_func,
    flash_attn_varlen_kvpacked_func as flash_attn_unpadded_kvpacked_func,
)
