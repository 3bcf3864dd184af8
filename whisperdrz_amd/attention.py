"""Drop-in attention entry points backed by the gfx950 HIP kernels in libwdrz_attn.so.

Two functions mirror the reference's two attention seams, with the same names, argument
meaning and output layout:

* :func:`flash_attn_with_kvcache` — the cached decoder path. Same signature as the dispatcher
  at reference ``src/whisperdrz/model.py:88-95`` and the semantics of its torch fallback
  ``_sdpa_attn_with_kvcache`` (``model.py:20-76``): in-place K/V append at ``cache_seqlens``,
  bottom-right causal mask over the slot, ``cache_batch_idx`` slot mapping; cross-attention
  (``k is None``) reads every cache row.
* :func:`scaled_dot_product_attention` — the dense path used by
  ``MultiHeadAttention.qkv_attention`` (``model.py:276-298``, the SDPA call at 288-296), for the
  encoder (non-causal, L=1500) and the uncached decoder (top-left causal).

There is deliberately no CPU or torch fallback here: CPU tensors, unsupported shapes and a
missing library raise. The reference keeps its own fallback for CPU tensors (its dispatcher
only routes ``q.is_cuda`` calls to the accelerated implementation).
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib

__all__ = [
    "flash_attn_with_kvcache",
    "scaled_dot_product_attention",
    "qkv_attention",
    "kvcache_workspace_size",
    "WorkspaceCache",
]

_DTYPES = {torch.float32: _lib.WDRZ_F32, torch.float16: _lib.WDRZ_F16, torch.bfloat16: _lib.WDRZ_BF16}
HEAD_DIM = 64


def _dtype_code(t: torch.Tensor, name: str) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"{name}: dtype {t.dtype} is not supported (float32, float16, bfloat16)") from None


def _check_cuda(name: str, t: torch.Tensor, device: torch.device) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise RuntimeError(
            f"{name} is on {t.device}: whisperdrz_amd runs on the GPU only (the reference keeps "
            "its torch fallback for CPU tensors)"
        )
    if t.device != device:
        raise RuntimeError(f"{name} is on {t.device}, expected {device}")


def _stream_handle() -> int:
    return torch.cuda.current_stream().cuda_stream


def _raise(rc: int, what: str) -> None:
    msg = _lib.last_error()
    if rc == _lib.WDRZ_EUNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    if rc == _lib.WDRZ_EINVAL or rc == _lib.WDRZ_EWORKSPACE:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


class WorkspaceCache:
    """Per-(device, stream) split-KV workspace, grown on demand and then reused.

    The workspace holds per-row arrival counters that must be zero before a call; every call
    leaves them zero again, so a buffer is zero-filled once, when it is allocated. Calls on
    one stream are ordered, so they can share a buffer; calls on different streams (e.g. the
    reference's side ``prefill_stream``) get different buffers. Call :meth:`reserve` before
    capturing a hipGraph so no allocation happens inside capture.
    """

    def __init__(self) -> None:
        self._bufs: dict[tuple[int, int], torch.Tensor] = {}

    def get(self, device: torch.device, nbytes: int) -> Optional[torch.Tensor]:
        if nbytes <= 0:
            return None
        key = (device.index if device.index is not None else torch.cuda.current_device(), _stream_handle())
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf

    def reserve(self, device: torch.device, nbytes: int) -> None:
        self.get(device, nbytes)

    def clear(self) -> None:
        self._bufs.clear()


_WORKSPACES = WorkspaceCache()


def kvcache_workspace_size(batch: int, sq: int, n_heads: int, head_dim: int, max_seq: int) -> int:
    """Bytes of split-KV workspace :func:`flash_attn_with_kvcache` needs for these sizes."""
    return int(_lib.load().wdrz_attn_kvcache_workspace_size(batch, sq, n_heads, head_dim, max_seq))


def _as_int32(name: str, t, B: int, device: torch.device) -> torch.Tensor:
    if isinstance(t, int):
        return torch.full((B,), t, dtype=torch.int32, device=device)
    _check_cuda(name, t, device)
    if t.dim() != 1 or t.shape[0] != B:
        raise ValueError(f"{name} must have shape [{B}], got {tuple(t.shape)}")
    if t.dtype != torch.int32:
        if t.dtype not in (torch.int64, torch.int16, torch.uint8, torch.int8):
            raise TypeError(f"{name} must be an integer tensor, got {t.dtype}")
        t = t.to(torch.int32)
    if t.stride(0) != 1:
        t = t.contiguous()
    return t


def flash_attn_with_kvcache(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k: Optional[torch.Tensor] = None,
    v: Optional[torch.Tensor] = None,
    cache_seqlens=None,
    cache_batch_idx: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
    causal: bool = False,
    *,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Attention of ``q`` against a slot KV cache (reference ``model.py:20-95``).

    ``out`` and ``workspace`` are keyword-only extensions: a preallocated output, and a
    caller-owned split-KV workspace (zero-filled before its first use; see
    :func:`kvcache_workspace_size`). Without ``workspace`` a per-stream cached one is used.

    Shapes: ``q`` ``[B, sq, H, D]``; ``k_cache``/``v_cache`` ``[n_slots, Lmax, H, D]`` (any
    strides with a contiguous last dim, e.g. head-major storage viewed as slot-major);
    ``k``/``v`` ``[B, sq, H, D]``; ``cache_seqlens`` int32 ``[B]`` (pre-append lengths);
    ``cache_batch_idx`` int32 ``[B]`` batch row -> slot. Returns ``[B, sq, H, D]`` in q's dtype.

    With ``k``/``v`` given they are written in place at rows ``cache_seqlens[b] + t`` of slot
    ``cache_batch_idx[b]`` and query ``t`` attends keys ``j <= cache_seqlens[b] + t``; the
    lengths themselves are not modified (the caller bumps them, ``model.py:602-607``). Without
    them the attention is non-causal over all ``Lmax`` rows. As in the reference fallback the
    mask follows from whether ``k`` is given; ``causal`` is accepted for signature parity.
    """
    lib = _lib.load()
    device = q.device
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        _check_cuda(name, t, device)
    if q.dim() != 4 or k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError("q, k_cache and v_cache must be 4-D ([B, sq, H, D] / [n_slots, Lmax, H, D])")
    B, sq, H, D = q.shape
    S, Lmax, Hc, Dc = k_cache.shape
    if tuple(v_cache.shape) != (S, Lmax, Hc, Dc):
        raise ValueError(f"v_cache shape {tuple(v_cache.shape)} != k_cache shape {tuple(k_cache.shape)}")
    if (Hc, Dc) != (H, D):
        raise ValueError(f"cache heads/head_dim {(Hc, Dc)} do not match q {(H, D)}")
    dt = _dtype_code(q, "q")
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise TypeError("k_cache and v_cache must have q's dtype")
    has_new = k is not None or v is not None
    if has_new:
        if k is None or v is None:
            raise ValueError("k and v must be given together")
        _check_cuda("k", k, device)
        _check_cuda("v", v, device)
        if tuple(k.shape) != (B, sq, H, D) or tuple(v.shape) != (B, sq, H, D):
            raise ValueError(f"k/v must have shape {(B, sq, H, D)}")
        if k.dtype != q.dtype or v.dtype != q.dtype:
            raise TypeError("k and v must have q's dtype")
        if cache_seqlens is None:
            raise ValueError("cache_seqlens is required when k/v are given")
        seqlens = _as_int32("cache_seqlens", cache_seqlens, B, device)
    else:
        seqlens = None
    bidx = None if cache_batch_idx is None else _as_int32("cache_batch_idx", cache_batch_idx, B, device)
    if _lib.debug_mode():  # host copies of the metadata: debugging runs only, not graph capture
        from .debug import check_kvcache_metadata

        check_kvcache_metadata(seqlens.cpu().numpy() if seqlens is not None else None,
                               bidx.cpu().numpy() if bidx is not None else None, sq, S, Lmax, has_new)
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    if out is None:
        out = torch.empty((B, sq, H, D), dtype=q.dtype, device=device)
    else:
        _check_cuda("out", out, device)
        if tuple(out.shape) != (B, sq, H, D) or out.dtype != q.dtype:
            raise ValueError("out must match q's shape and dtype")
    if B == 0 or sq == 0:
        return out
    nbytes = int(lib.wdrz_attn_kvcache_workspace_size(B, sq, H, D, Lmax))
    if nbytes > 0:
        if workspace is None:
            workspace = _WORKSPACES.get(device, nbytes)
        elif workspace.numel() * workspace.element_size() < nbytes:
            raise ValueError(f"workspace too small: need {nbytes} bytes")
    ws_ptr = workspace.data_ptr() if (nbytes > 0 and workspace is not None) else None
    ws_bytes = workspace.numel() * workspace.element_size() if ws_ptr else 0
    rc = lib.wdrz_attn_kvcache(
        dt,
        q.data_ptr(),
        k_cache.data_ptr(),
        v_cache.data_ptr(),
        k.data_ptr() if has_new else None,
        v.data_ptr() if has_new else None,
        seqlens.data_ptr() if seqlens is not None else None,
        bidx.data_ptr() if bidx is not None else None,
        out.data_ptr(),
        B, sq, H, D, S, Lmax,
        _lib.strides4(q.stride()),
        _lib.strides4(k_cache.stride()),
        _lib.strides4(v_cache.stride()),
        _lib.strides4(k.stride() if has_new else (0, 0, 0, 1)),
        _lib.strides4(v.stride() if has_new else (0, 0, 0, 1)),
        _lib.strides4(out.stride()),
        float(softmax_scale),
        int(bool(causal)),
        ws_ptr,
        ws_bytes,
        _stream_handle(),
    )
    if rc != _lib.WDRZ_OK:
        _raise(rc, "flash_attn_with_kvcache")
    return out


def scaled_dot_product_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attn_mask: Optional[torch.Tensor] = None,
    dropout_p: float = 0.0,
    is_causal: bool = False,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """``F.scaled_dot_product_attention`` for ``[B, H, L, 64]`` inputs (reference ``model.py:288-296``).

    Inputs may be strided views (the reference passes rearranged ``[B, T, H*D]`` projections).
    The result is a ``[B, H, Lq, D]`` view of ``[B, Lq, H, D]`` storage, so the reference's
    ``rearrange(out, "B h T d -> B T (h d)")`` that follows is free. ``is_causal`` is torch's
    top-left aligned mask. ``attn_mask`` and dropout are not supported (the reference passes
    neither at inference).
    """
    if attn_mask is not None:
        raise NotImplementedError("attn_mask is not supported (the reference passes None)")
    if dropout_p != 0.0:
        raise NotImplementedError("dropout is not supported at inference")
    lib = _lib.load()
    device = query.device
    for name, t in (("query", query), ("key", key), ("value", value)):
        _check_cuda(name, t, device)
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise ValueError("query/key/value must be 4-D [B, H, L, D]")
    B, H, Lq, D = query.shape
    Bk, Hk, Lk, Dk = key.shape
    if (Bk, Hk, Dk) != (B, H, D) or tuple(value.shape) != (B, H, Lk, D):
        raise ValueError(
            f"shape mismatch: query {tuple(query.shape)}, key {tuple(key.shape)}, value {tuple(value.shape)}"
        )
    dt = _dtype_code(query, "query")
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise TypeError("query, key and value must share a dtype")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty((B, Lq, H, D), dtype=query.dtype, device=device).permute(0, 2, 1, 3)
    if B == 0 or Lq == 0:
        return out
    if Lk == 0:
        raise ValueError("key length must be >= 1")
    rc = lib.wdrz_attn_fwd(
        dt,
        query.data_ptr(),
        key.data_ptr(),
        value.data_ptr(),
        out.data_ptr(),
        B, H, Lq, Lk, D,
        _lib.strides4(query.stride()),
        _lib.strides4(key.stride()),
        _lib.strides4(value.stride()),
        _lib.strides4(out.stride()),
        float(scale),
        int(bool(is_causal)),
        _stream_handle(),
    )
    if rc != _lib.WDRZ_OK:
        _raise(rc, "scaled_dot_product_attention")
    return out


def qkv_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, n_head: int, causal: bool = False) -> torch.Tensor:
    """Attention core of ``MultiHeadAttention.qkv_attention`` (reference ``model.py:276-298``).

    ``q``, ``k``, ``v`` are the ``[B, T, n_head*64]`` projection outputs; returns
    ``[B, Tq, n_head*64]`` before the output projection. The scale is ``(D**-0.25)**2`` and the
    mask is causal only when ``causal and Tq > 1`` (``model.py:280-294``).
    """
    B, Tq, n_state = q.shape
    D = n_state // n_head
    scale = D ** -0.25
    qh = q.view(B, Tq, n_head, D).permute(0, 2, 1, 3)
    kh = k.view(k.shape[0], k.shape[1], n_head, D).permute(0, 2, 1, 3)
    vh = v.view(v.shape[0], v.shape[1], n_head, D).permute(0, 2, 1, 3)
    out = scaled_dot_product_attention(qh, kh, vh, is_causal=causal and Tq > 1, scale=scale * scale)
    return out.permute(0, 2, 1, 3).reshape(B, Tq, n_state)
