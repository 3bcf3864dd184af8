"""whisperdrz_amd — MI355X-native (gfx950) attention hot path for WhisperDRZ.

Drop-in entry points for the reference's two attention seams (src/whisperdrz/model.py:88-95 and
model.py:288-296), backed by hand-written HIP kernels in libwdrz_attn.so, plus the slot KV cache
(model.py:98-192) and the decode-step plumbing around them.
"""
from . import _lib
from .attention import (
    WorkspaceCache,
    flash_attn_with_kvcache,
    kvcache_workspace_size,
    qkv_attention,
    scaled_dot_product_attention,
)

HAS_WDRZ = _lib.available()

__all__ = [
    "HAS_WDRZ",
    "WorkspaceCache",
    "flash_attn_with_kvcache",
    "kvcache_workspace_size",
    "qkv_attention",
    "scaled_dot_product_attention",
]
