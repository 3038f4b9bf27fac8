"""flash_attn_npu_v2 on MI355X: the v2 FlashAttention Python API (forward).

Same module, function and keyword names as the reference package
(flash_attn_npu_v2/__init__.py:12-21 there). The reference picks its backend
from the Ascend device name and raises elsewhere; here there is one backend,
the HIP kernels for gfx950 loaded by fa_mi355x.
"""
__version__ = "0.1.1"

from .interface import (  # noqa: F401
    flash_attn_func,
    flash_attn_kvpacked_func,
    flash_attn_qkvpacked_func,
    flash_attn_varlen_func,
    flash_attn_varlen_kvpacked_func,
    flash_attn_varlen_qkvpacked_func,
    flash_attn_with_kvcache,
)
