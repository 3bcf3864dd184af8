"""Opt-in host-side checks of cached-attention metadata, and the torch A/B switch.

``WDRZ_DEBUG=1`` makes :func:`whisperdrz_amd.flash_attn_with_kvcache` copy the slot ids and
pre-append lengths of every call to the host and check them with :func:`check_kvcache_metadata`
before launching (it also selects ``libwdrz_attn_debug.so``, whose C layer repeats the checks).
The release path never reads device memory from the host, so it stays capture-safe; these checks
do, so they are for debugging runs only.

``WDRZ_FORCE_TORCH=1`` makes the import-time probe :func:`probe` (and ``HAS_WDRZ``) report the
HIP library as unavailable, so a caller that gates on it the way the reference gates on
``HAS_FLASH_ATTN`` (src/whisperdrz/model.py:79-95) runs its own torch path: an A/B switch for the
reference's torch fallback, like ``flash_kernel(flash=False)`` at src/whisperdrz/utils.py:48-62.
"""
from __future__ import annotations

import os
from typing import Optional

import numpy as np

__all__ = ["check_kvcache_metadata", "force_torch", "probe"]


def force_torch() -> bool:
    """True when WDRZ_FORCE_TORCH asks callers to use their torch path."""
    return os.environ.get("WDRZ_FORCE_TORCH", "0") not in ("", "0")


def probe() -> bool:
    """Whether callers should route attention to the HIP library: it loads and
    WDRZ_FORCE_TORCH is not set (evaluated at call time)."""
    from . import _lib

    return not force_torch() and _lib.available()


def check_kvcache_metadata(cache_seqlens: Optional[np.ndarray], cache_batch_idx: Optional[np.ndarray], sq: int,
                           n_slots: int, max_seq: int, append: bool) -> None:
    """Check the metadata of one ``flash_attn_with_kvcache`` call (host arrays).

    Raises ``ValueError`` for a row whose slot id is outside ``[0, n_slots)`` or, with an
    append, whose region ``[cs, cs + sq)`` leaves the cache. Rows naming the same slot (the
    padded rows of a bucketed decode graph, transcriber.py:76-78, 165-169) are valid: the kernels
    apply their appends in batch order, the last row covering a position winning, as the
    fallback's loop does (model.py:51-54).
    """
    if cache_batch_idx is None and cache_seqlens is None:
        return
    B = len(cache_batch_idx) if cache_batch_idx is not None else len(cache_seqlens)
    slots = np.arange(B) if cache_batch_idx is None else np.asarray(cache_batch_idx, dtype=np.int64)
    bad = np.flatnonzero((slots < 0) | (slots >= n_slots))
    if bad.size:
        i = int(bad[0])
        raise ValueError(f"row {i} names slot {int(slots[i])} outside [0, {n_slots})")
    if not append:
        return
    cs = np.asarray(cache_seqlens, dtype=np.int64)
    bad = np.flatnonzero((cs < 0) | (cs + sq > max_seq))
    if bad.size:
        i = int(bad[0])
        raise ValueError(f"row {i} appends [{int(cs[i])}, {int(cs[i]) + sq}) outside the cache [0, {max_seq})")
