"""DTW alignment inputs on the GPU, backed by the gfx950 kernels in libwdrz_attn.so.

:func:`compute_attention` mirrors ``CrossAttnCapture.compute_attention(head_mask)``
(``src/whisperdrz/dtw_align.py:553-586``): the raw Q K^T of the selected alignment heads, read in
place from the captured per-layer query / key projections.

:func:`dtw_prep_batch` mirrors the reference's batched prep ``_dtw_prep_batch(full_weights, actual_lens, audio_caps,
medfilt_width=7)`` (``src/whisperdrz/dtw_align.py:700-753``): capped row softmax, column
mean/std normalisation over each chunk's valid text rows, width-``medfilt_width`` median filter
along the audio axis (reflect padding), mean over the alignment heads, slice to the largest cap,
one device->host copy into a reused pinned buffer.

There is no CPU fallback: CPU tensors and a missing library raise.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np
import torch

from . import _lib
from .attention import WorkspaceCache, _check_cuda, _raise, _stream_handle

__all__ = ["compute_attention", "dtw_attention_prep", "dtw_prep", "median_filter", "dtw_prep_batch", "dtw_prep_workspace_size"]

_QK_DTYPES = {torch.bfloat16: _lib.WDRZ_BF16, torch.float16: _lib.WDRZ_F16}

# The prep's workspace holds no state between calls; it is kept apart from the split-KV
# workspace, whose counters must stay zero.
_DTW_WORKSPACES = WorkspaceCache()
_PINNED: dict[tuple, torch.Tensor] = {}


class _Heads:
    """The selected heads' query / key slices as one set of per-head pointers with shared strides."""

    def __init__(self, q_out, k_out, head_mask):
        mask = torch.as_tensor(head_mask)
        n_heads = int(mask.shape[1])
        sel = mask.nonzero().tolist()
        if not sel:
            raise ValueError("head_mask selects no heads")
        q_views, k_views = [], []
        for layer, head in sel:
            q, k = q_out[layer], k_out[layer]
            if q is None or k is None:
                raise ValueError(f"layer {layer} has no captured projection")
            B, T, width = q.shape
            D = width // n_heads
            q_views.append(q.view(B, T, n_heads, D)[:, :, head])
            k_views.append(k.view(k.shape[0], k.shape[1], n_heads, D)[:, :, head])
        q0, k0 = q_views[0], k_views[0]
        self.device = q0.device
        _check_cuda("q_out", q0, self.device)
        if q0.dtype not in _QK_DTYPES:
            raise TypeError(f"q_out: dtype {q0.dtype} is not supported (bfloat16, float16)")
        self.B, self.T, self.D = (int(x) for x in q0.shape)
        self.A = int(k0.shape[1])
        dev = self.device
        same = all(v.stride() == q0.stride() and v.dtype == q0.dtype and v.device == dev for v in q_views) and all(
            v.stride() == k0.stride() and v.dtype == q0.dtype and v.device == dev and v.shape[1] == self.A
            for v in k_views
        )
        if not same:  # heads from differently laid-out captures: give them one layout
            q_views = [v.contiguous() for v in q_views]
            k_views = [v.to(q0.dtype).contiguous() for v in k_views]
        self.views = (q_views, k_views)  # keeps the copies alive for the call
        self.H = len(sel)
        self.dtype = _QK_DTYPES[q0.dtype]
        self.qp = (_lib.ctypes.c_void_p * self.H)(*[v.data_ptr() for v in q_views])
        self.kp = (_lib.ctypes.c_void_p * self.H)(*[v.data_ptr() for v in k_views])
        self.qs = (_lib.ctypes.c_int64 * 3)(*q_views[0].stride())
        self.ks = (_lib.ctypes.c_int64 * 3)(*k_views[0].stride())
        self.scale = float(self.D) ** -0.25  # dtw_align.py:561


def compute_attention(q_out, k_out, head_mask) -> torch.Tensor:
    """Drop-in for ``CrossAttnCapture.compute_attention`` (dtw_align.py:553-586).

    q_out / k_out: the captured ``cross_attn.query`` / ``cross_attn.key`` outputs per decoder
    layer (``[B, T_text, n_heads*64]`` / ``[B, T_audio, n_heads*64]``, bf16 or fp16 on the GPU;
    ``None`` for layers without a selected head). head_mask: bool ``[n_layers, n_heads]``.
    Returns fp32 ``[B, n_selected, T_text, T_audio]``, or ``[n_selected, T_text, T_audio]`` when
    B == 1, as the reference does. Each head's slice is read in place; no stacked copies.
    """
    hd = _Heads(q_out, k_out, head_mask)
    B, H, T, A = hd.B, hd.H, hd.T, hd.A
    out = torch.empty((B, H, T, A), dtype=torch.float32, device=hd.device)
    rc = _lib.load().wdrz_dtw_qk(
        hd.dtype, hd.qp, hd.qs, hd.kp, hd.ks, out.data_ptr(), _lib.strides4(out.stride()),
        B, H, T, A, hd.D, hd.scale, _stream_handle(),
    )
    if rc != _lib.WDRZ_OK:
        _raise(rc, "compute_attention")
    return out[0] if B == 1 else out


def dtw_attention_prep(q_out, k_out, head_mask, actual_lens: Sequence[int], audio_caps: Sequence[int],
                       medfilt_width: int = 7) -> torch.Tensor:
    """``dtw_prep(compute_attention(q_out, k_out, head_mask), actual_lens, audio_caps)`` in one
    pass over the projections: the scores are recomputed on the matrix cores inside the prep
    instead of being stored (dtw_align.py:1184-1197). Returns the device tensor
    ``[B, T_text, max_audio_cap]`` (fp32). T_audio <= 1536."""
    hd = _Heads(q_out, k_out, head_mask)
    B, H, T, A = hd.B, hd.H, hd.T, hd.A
    lens = [int(x) for x in actual_lens]
    caps = [int(x) for x in audio_caps]
    if len(lens) != B or len(caps) != B:
        raise ValueError(f"actual_lens / audio_caps must have {B} entries")
    C = len(range(A)[: max(caps)])
    out = torch.empty((B, T, C), dtype=torch.float32, device=hd.device)
    if T == 0 or C == 0:
        return out
    meta = torch.tensor([lens, caps], dtype=torch.int32).pin_memory().to(hd.device, non_blocking=True)
    nbytes = dtw_prep_workspace_size(B, H, T, A)
    ws = _DTW_WORKSPACES.get(hd.device, nbytes)
    rc = _lib.load().wdrz_dtw_attention_prep(
        hd.dtype, hd.qp, hd.qs, hd.kp, hd.ks, hd.scale, meta[0].data_ptr(), meta[1].data_ptr(),
        out.data_ptr(), (_lib.ctypes.c_int64 * 3)(*out.stride()), B, H, T, A, hd.D, C, int(medfilt_width),
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, _stream_handle(),
    )
    if rc != _lib.WDRZ_OK:
        _raise(rc, "dtw_attention_prep")
    return out


def median_filter(x: torch.Tensor, width: int) -> torch.Tensor:
    """Drop-in for ``median_filter(x, width)`` (dtw_align.py:156-167): the median of each
    ``width``-wide window along the last axis, reflect padding, same shape and dtype as ``x``.
    ``width`` is 1 or odd <= 15; a last axis no longer than ``width // 2`` is returned as it is.
    Other float dtypes are filtered in fp32 (a median selects one input, so the conversion back
    is exact)."""
    if not isinstance(x, torch.Tensor):
        raise TypeError("x must be a torch.Tensor")
    _check_cuda("x", x, x.device)
    if not x.is_floating_point():
        raise TypeError(f"x: dtype {x.dtype} is not a floating-point type")
    if x.dim() == 0:
        raise ValueError("x must have at least one axis")
    N = int(x.shape[-1])
    rows = x.numel() // N if N else 0
    src = x.reshape(rows, N) if N else x.reshape(0, 0)
    src = src.to(torch.float32)
    if src.stride(-1) != 1:
        src = src.contiguous()
    out = torch.empty((rows, N), dtype=torch.float32, device=x.device)
    rc = _lib.load().wdrz_median_filter(src.data_ptr(), src.stride(0) if rows else N, out.data_ptr(), N, rows, N,
                                        int(width), _stream_handle())
    if rc != _lib.WDRZ_OK:
        _raise(rc, "median_filter")
    return out.view(x.shape).to(x.dtype)


def dtw_prep_workspace_size(B: int, H: int, T: int, A: int) -> int:
    """Bytes of device workspace :func:`dtw_prep` needs for a [B, H, T, A] score tensor."""
    return int(_lib.load().wdrz_dtw_prep_workspace_size(B, H, T, A))


def _kernel_ready(w: torch.Tensor) -> torch.Tensor:
    """The kernels need unit stride along the audio axis (compute_attention's output has it)."""
    return w if w.stride(-1) == 1 else w.contiguous()


def dtw_prep(
    full_weights: torch.Tensor,
    actual_lens: Sequence[int],
    audio_caps: Sequence[int],
    medfilt_width: int = 7,
) -> torch.Tensor:
    """The prep of ``_dtw_prep_batch`` without the host copy: returns the device tensor
    ``[B, T_text_pad, max_audio_cap]`` (fp32).

    full_weights: fp32 ``[B, H, T_text_pad, T_audio]`` on the GPU (raw Q K^T of the alignment
    heads). ``actual_lens[b]`` rows enter the column statistics; columns ``>= audio_caps[b]``
    are masked out of the softmax (dtw_align.py:720-738).
    """
    w = full_weights
    if not isinstance(w, torch.Tensor):
        raise TypeError("full_weights must be a torch.Tensor")
    if w.dim() != 4:
        raise ValueError(f"full_weights must be [B, H, T_text, T_audio], got shape {tuple(w.shape)}")
    if w.dtype != torch.float32:
        raise TypeError(f"full_weights: dtype {w.dtype} is not supported (float32, as compute_attention gives)")
    device = w.device
    _check_cuda("full_weights", w, device)
    B, H, T, A = (int(x) for x in w.shape)
    lens = [int(x) for x in actual_lens]
    caps = [int(x) for x in audio_caps]
    if len(lens) != B or len(caps) != B:
        raise ValueError(f"actual_lens / audio_caps must have {B} entries")
    if B == 0:
        raise ValueError("empty batch (the reference's max() over no caps raises too)")
    # matrix[:, :, :max_audio_cap] (dtw_align.py:746), with Python's slice semantics.
    C = len(range(A)[: max(caps)])
    out = torch.empty((B, T, C), dtype=torch.float32, device=device)
    if T == 0 or C == 0:
        return out
    w = _kernel_ready(w)
    # One small host->device copy from pinned memory, ordered on the current stream.
    meta = torch.tensor([lens, caps], dtype=torch.int32).pin_memory().to(device, non_blocking=True)
    lens_t, caps_t = meta[0], meta[1]
    lib = _lib.load()
    nbytes = dtw_prep_workspace_size(B, H, T, A)
    ws = _DTW_WORKSPACES.get(device, nbytes)
    ws_ptr = ws.data_ptr() if ws is not None else None
    rc = lib.wdrz_dtw_prep(
        w.data_ptr(), _lib.strides4(w.stride()), lens_t.data_ptr(), caps_t.data_ptr(),
        out.data_ptr(), (_lib.ctypes.c_int64 * 3)(*out.stride()),
        B, H, T, A, C, int(medfilt_width), ws_ptr, ws.numel() if ws is not None else 0,
        _stream_handle(),
    )
    if rc != _lib.WDRZ_OK:
        _raise(rc, "dtw_prep")
    return out


def dtw_prep_batch(
    full_weights: torch.Tensor,
    actual_lens: Sequence[int],
    audio_caps: Sequence[int],
    medfilt_width: int = 7,
) -> np.ndarray:
    """Drop-in for ``_dtw_prep_batch`` (dtw_align.py:700-753): the prep on the GPU, then ONE
    device->host copy into a pinned buffer reused per shape. As in the reference, the returned
    array shares that buffer, so it is overwritten by the next call of the same shape."""
    matrix = dtw_prep(full_weights, actual_lens, audio_caps, medfilt_width)
    key = (tuple(matrix.shape), matrix.dtype)
    host = _PINNED.get(key)
    if host is None:
        host = torch.empty(matrix.shape, dtype=matrix.dtype, pin_memory=True)
        _PINNED[key] = host
    host.copy_(matrix, non_blocking=True)
    torch.cuda.synchronize(matrix.device)
    return host.numpy()


# The reference's private name, for a one-line swap at dtw_align.py:1197.
_dtw_prep_batch = dtw_prep_batch
