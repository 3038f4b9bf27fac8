"""flash_attn_npu_v3 on MI355X: the v3 FlashAttention Python API (forward).

Same names as the reference package (flash_attn_npu_v3/__init__.py:18-28
there), without the device-name dispatch: one backend, the gfx950 kernels
loaded by fa_mi355x.
"""
__version__ = "0.1.1"

from .interface import (  # noqa: F401
    flash_attn_combine,
    flash_attn_func,
    flash_attn_varlen_func,
    flash_attn_with_kvcache,
    get_scheduler_metadata,
)
