"""whisperdrz_amd — MI355X-native (gfx950) attention hot path for WhisperDRZ.

Drop-in entry points for the reference's two attention seams (src/whisperdrz/model.py:88-95 and
model.py:288-296), backed by hand-written HIP kernels in libwdrz_attn.so, plus the slot KV cache
(model.py:98-192), the decode-step plumbing around them, the DTW alignment inputs
(dtw_align.py:553-586, 700-753) and the log-mel front end (audio.py:81-156).
"""
from . import _lib
from .attention import (
    WorkspaceCache,
    flash_attn_with_kvcache,
    kvcache_workspace_size,
    qkv_attention,
    scaled_dot_product_attention,
)
from .audio import LogMelSpectrogram, log_mel_spectrogram
from .decode_ops import (add_layernorm_, add_layernorm_partials_, layer_norm, linear, linear_gelu, linear_partials,
                         masked_argmax)
from .dtw import (compute_attention, dtw_attention_prep, dtw_prep, dtw_prep_batch, dtw_prep_workspace_size,
                  median_filter)

from .debug import check_kvcache_metadata, force_torch, probe

# Import-time probe, the counterpart of the reference's HAS_FLASH_ATTN (model.py:79-84): true when
# the HIP library loads and WDRZ_FORCE_TORCH is not set.
HAS_WDRZ = probe()

__all__ = [
    "HAS_WDRZ",
    "check_kvcache_metadata",
    "force_torch",
    "probe",
    "LogMelSpectrogram",
    "add_layernorm_",
    "add_layernorm_partials_",
    "layer_norm",
    "linear",
    "linear_gelu",
    "linear_partials",
    "masked_argmax",
    "log_mel_spectrogram",
    "compute_attention",
    "dtw_attention_prep",
    "median_filter",
    "dtw_prep",
    "dtw_prep_batch",
    "dtw_prep_workspace_size",
    "WorkspaceCache",
    "flash_attn_with_kvcache",
    "kvcache_workspace_size",
    "qkv_attention",
    "scaled_dot_product_attention",
]
