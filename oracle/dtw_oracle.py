"""CPU restatement of the reference's DTW alignment prep — TEST INFRASTRUCTURE ONLY.

Imported only by tests/ and bench.py's cpu_baseline leg, as the checker or the timed CPU
baseline. The product (whisperdrz_amd) never imports it.

Covers two steps that run between the decoder forward and the numba DTW:

  compute_attention_ref   CrossAttnCapture.compute_attention (src/whisperdrz/dtw_align.py:553-586):
                          raw Q K^T of the selected alignment heads, no softmax, fp32, each
                          operand scaled by head_dim**-0.25.
  dtw_prep_ref            _dtw_prep_batch (dtw_align.py:700-753) without the device->host copy:
                          capped row softmax, per-column mean/std over the valid text rows,
                          median filter along the audio axis, mean over heads, slice to the
                          largest cap.

Parity is pinned in tests/test_dtw_oracle.py against independent formulations:
scipy.ndimage.median_filter (mode="mirror" is torch's "reflect" padding), torch.softmax +
torch.std_mean (the reference's single-chunk path, dtw_align.py:772-780) and closed-form
invariants (zero-mean / unit-variance columns before the filter, exact zeros in masked columns).
"""
from __future__ import annotations

import numpy as np


def median_filter_ref(x: np.ndarray, width: int) -> np.ndarray:
    """Median filter along the last axis with reflect padding (dtw_align.py:65-78, 156-167).

    pad = width // 2; a last axis of length <= pad is returned unchanged (dtw_align.py:68-69).
    Padding is torch's "reflect" (the edge sample is not repeated): x[-1] -> x[1].
    The median is element width // 2 of the sorted window.
    """
    x = np.asarray(x)
    pad = width // 2
    if x.shape[-1] <= pad:
        return x.copy()
    widths = [(0, 0)] * (x.ndim - 1) + [(pad, pad)]
    xp = np.pad(x, widths, mode="reflect")
    win = np.lib.stride_tricks.sliding_window_view(xp, width, axis=-1)
    return np.sort(win, axis=-1)[..., width // 2]


def dtw_prep_ref(full_weights, actual_lens, audio_caps, medfilt_width: int = 7,
                 dtype=np.float64) -> np.ndarray:
    """Restatement of _dtw_prep_batch (dtw_align.py:700-753) in `dtype` (float64 by default).

    full_weights: [B, H, T, A] raw scores. Returns [B, T, max(audio_caps)].
      1. columns >= audio_caps[b] are masked to -inf and each row is softmaxed
         (dtw_align.py:724-727); a cap of 0 leaves a row of all -inf, whose softmax is NaN;
      2. over the rows t < actual_lens[b], with n = actual_lens[b]:
         mean = sum / n, var = sum((w - mean)^2) / n, std = sqrt(max(var, 1e-12)),
         and EVERY row is normalised as (w - mean) / std (dtw_align.py:729-738);
      3. median filter of width `medfilt_width` along the audio axis when it is > 1
         (dtw_align.py:742-743);
      4. mean over heads, slice to the largest cap (dtw_align.py:745-746).
    """
    w = np.asarray(full_weights, dtype=dtype)
    B, H, T, A = w.shape
    lens = np.asarray(actual_lens, dtype=np.int64).reshape(B)
    caps = np.asarray(audio_caps, dtype=np.int64).reshape(B)
    max_cap = int(caps.max()) if B else 0
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        audio_mask = np.arange(A)[None, :] < caps[:, None]  # [B, A]
        w = np.where(audio_mask[:, None, None, :], w, -np.inf)
        m = np.max(w, axis=-1, keepdims=True)
        e = np.exp(w - m)  # all -inf row: exp(nan) = nan, as torch.softmax gives
        w = e / np.sum(e, axis=-1, keepdims=True)

        text_mask = (np.arange(T)[None, :] < lens[:, None]).astype(dtype)[:, None, :, None]
        n = lens.astype(dtype).reshape(B, 1, 1, 1)
        mean = np.sum(w * text_mask, axis=-2, keepdims=True) / n
        var = np.sum(((w - mean) ** 2) * text_mask, axis=-2, keepdims=True) / n
        var = np.where(np.isnan(var), var, np.maximum(var, 1e-12))  # clamp_min keeps NaN
        w = (w - mean) / np.sqrt(var)

        if medfilt_width > 1:
            w = median_filter_ref(w, medfilt_width)
        return w.mean(axis=1)[:, :, :max_cap]


def compute_attention_ref(q_heads, k_heads, head_dim: int = 64) -> np.ndarray:
    """Q K^T of the selected heads, in float64 (dtw_align.py:553-586).

    q_heads: [n_sel, B, T_text, D], k_heads: [n_sel, B, T_audio, D] (the gathered per-head
    slices). Each operand is scaled by head_dim**-0.25 (dtw_align.py:561). Returns
    [B, n_sel, T_text, T_audio] (the reference drops the batch axis when B == 1; callers lift it
    back, dtw_align.py:1185-1187, so the 4-D form is what the prep sees).
    """
    s = head_dim ** -0.25
    q = np.asarray(q_heads, dtype=np.float64) * s
    k = np.asarray(k_heads, dtype=np.float64) * s
    return np.swapaxes(np.matmul(q, np.swapaxes(k, -1, -2)), 0, 1)


def dtw_prep_torch(full_weights, actual_lens, audio_caps, medfilt_width: int = 7):
    """The same steps as dtw_prep_ref in torch fp32 ops (the reference's own op sequence,
    dtw_align.py:720-746, with the sort-based median filter of dtw_align.py:65-78 that the
    reference uses off-GPU), on whatever device `full_weights` is on. Used as the timed CPU
    baseline and, on a GPU tensor, as a full-size fp32 check."""
    import torch

    w = torch.as_tensor(full_weights, dtype=torch.float32)
    dev = w.device
    B, H, T, A = w.shape
    lens = torch.as_tensor(actual_lens, dtype=torch.long).to(dev)
    caps = torch.as_tensor(audio_caps, dtype=torch.long).to(dev)
    max_cap = int(caps.max())
    audio_mask = torch.arange(A, device=dev)[None, :] < caps[:, None]
    w = torch.softmax(w.masked_fill(~audio_mask[:, None, None, :], float("-inf")), dim=-1)
    text_mask = (torch.arange(T, device=dev)[None, :] < lens[:, None])[:, None, :, None].to(w.dtype)
    n = lens.view(B, 1, 1, 1).to(w.dtype)
    mean = (w * text_mask).sum(dim=-2, keepdim=True) / n
    var = (((w - mean) ** 2) * text_mask).sum(dim=-2, keepdim=True) / n
    w = (w - mean) / var.clamp_min(1e-12).sqrt()
    if medfilt_width > 1:
        w = median_filter_torch(w, medfilt_width)
    return w.mean(dim=1)[:, :, :max_cap].contiguous()


def median_filter_torch(x, width: int):
    """The reference's sort-based median filter (_median_filter_sort, dtw_align.py:63-78) in
    torch ops on whatever device ``x`` is on: reflect pad, unfold, sort, middle element."""
    import torch

    pad = width // 2
    if x.shape[-1] <= pad:
        return x
    flat = torch.nn.functional.pad(x.reshape(-1, 1, x.shape[-1]), (pad, pad), mode="reflect")
    return flat.unfold(-1, width, 1).sort(dim=-1).values[..., pad].reshape(x.shape)
