"""Whisper's log-mel front end on the GPU, backed by the gfx950 kernels in libwdrz_attn.so.

:class:`LogMelSpectrogram` mirrors the reference module of the same name
(``src/whisperdrz/audio.py:81-156``): same constructor arguments, same ``forward(waveform,
target_frames=None)`` over a 1-D waveform, a batch ``[B, N]`` or a list of waveforms, same
result (``[n_mels, frames]`` or ``[B, n_mels, frames]``, fp32, padded with -1.5 or truncated to
``target_frames``). It runs where the reference's transcriber runs its CPU module
(``transcriber.py:1091-1092``) and returns the mel already on the GPU.

There is no CPU fallback: a missing library raises; CPU waveforms are copied to the GPU.
"""
from __future__ import annotations

from typing import Optional, Sequence, Union

import torch

from . import _lib
from .attention import WorkspaceCache, _raise, _stream_handle

__all__ = ["LogMelSpectrogram", "log_mel_spectrogram", "log_mel_workspace_size"]

_MEL_WORKSPACES = WorkspaceCache()


def log_mel_workspace_size(batch: int, n_mels: int) -> int:
    return int(_lib.load().wdrz_log_mel_workspace_size(batch, n_mels))


def log_mel_spectrogram(audio: torch.Tensor, n_mels: int = 128, target_frames: Optional[int] = None,
                        device: Optional[torch.device] = None) -> torch.Tensor:
    """Log-mel of a waveform ``[N]`` or a batch ``[B, N]`` (fp32) on the GPU."""
    if not isinstance(audio, torch.Tensor):
        raise TypeError("audio must be a torch.Tensor")
    if device is None:
        device = audio.device if audio.is_cuda else torch.device("cuda", torch.cuda.current_device())
    single = audio.dim() == 1
    x = audio.reshape(1, -1) if single else audio
    if x.dim() != 2:
        raise ValueError(f"audio must be [N] or [B, N], got shape {tuple(audio.shape)}")
    x = x.to(device=device, dtype=torch.float32)
    if x.stride(-1) != 1:
        x = x.contiguous()
    B, N = (int(v) for v in x.shape)
    n_frames = N // 160
    frames = n_frames if target_frames is None else int(target_frames)
    out = torch.empty((B, n_mels, frames), dtype=torch.float32, device=device)
    nbytes = log_mel_workspace_size(B, n_mels)
    ws = _MEL_WORKSPACES.get(device, nbytes)
    rc = _lib.load().wdrz_log_mel(
        x.data_ptr(), B, N, x.stride(0), out.data_ptr(), (_lib.ctypes.c_int64 * 3)(*out.stride()),
        n_mels, -1 if target_frames is None else frames, ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0, _stream_handle(),
    )
    if rc != _lib.WDRZ_OK:
        _raise(rc, "log_mel_spectrogram")
    return out[0] if single else out


class LogMelSpectrogram:
    """Drop-in for the reference's ``LogMelSpectrogram`` module (audio.py:81-156)."""

    def __init__(self, n_mels: int = 128, sample_rate: int = 16_000, n_fft: int = 400, hop_length: int = 160,
                 norm: str = "slaney", mel_scale: str = "slaney", device: Optional[torch.device] = None):
        if (sample_rate, n_fft, hop_length, norm, mel_scale) != (16_000, 400, 160, "slaney", "slaney"):
            raise NotImplementedError("only Whisper's front end (16 kHz, n_fft 400, hop 160, slaney) is built")
        self.n_mels = n_mels
        self.sample_rate = sample_rate
        self.n_fft = n_fft
        self.hop_length = hop_length
        self.device = device

    def forward(self, waveform: Union[torch.Tensor, Sequence[torch.Tensor]],
                target_frames: Optional[int] = None) -> torch.Tensor:
        if isinstance(waveform, (list, tuple)):
            # audio.py:110-116: each waveform on its own (lengths may differ), then stacked
            return torch.stack([self._single(w, target_frames) for w in waveform])
        if waveform.dim() == 1:
            return self._single(waveform, target_frames)
        # a batch: one launch for all rows (each row keeps its own window maximum)
        return log_mel_spectrogram(waveform, self.n_mels, target_frames, self.device)

    __call__ = forward

    def _single(self, audio: torch.Tensor, target_frames: Optional[int]) -> torch.Tensor:
        return log_mel_spectrogram(audio, self.n_mels, target_frames, self.device)
