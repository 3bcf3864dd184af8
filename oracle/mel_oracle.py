"""CPU restatement of the reference's log-mel front end — TEST INFRASTRUCTURE ONLY.

Imported only by tests/ and bench.py's cpu_baseline leg, as the checker or the timed CPU
baseline. The product (whisperdrz_amd) never imports it.

Restates LogMelSpectrogram (src/whisperdrz/audio.py:81-156): torch.stft (n_fft 400, hop 160,
periodic Hann window, center=True with reflect padding, one-sided), power of all frames but the
last, a slaney mel filterbank, log10 clamped at 1e-10, floor at (max - 8), (x + 4) / 4, and the
optional padding to target_frames with -1.5 / truncation (audio.py:128-139).

The filterbank comes from torchaudio.transforms.MelScale(norm="slaney", mel_scale="slaney")
(audio.py:97-103), a dependency the reference does not pin (pyproject.toml lists "torchaudio")
and that is absent here. Its published algorithm (torchaudio.functional.melscale_fbanks, the
same construction as librosa.filters.mel with htk=False, norm="slaney") is restated in
`mel_filterbank` and pinned in tests/test_mel_oracle.py by closed-form properties of the slaney
scale and the triangular, area-normalised filters; the STFT is pinned against torch.stft.
"""
from __future__ import annotations

import math

import numpy as np

SAMPLE_RATE = 16000
N_FFT = 400
HOP_LENGTH = 160

_F_SP = 200.0 / 3.0  # slaney: 3 mels per 200 Hz below 1 kHz
_MIN_LOG_HZ = 1000.0
_MIN_LOG_MEL = _MIN_LOG_HZ / _F_SP  # 15
_LOGSTEP = math.log(6.4) / 27.0  # log spacing above 1 kHz


def hz_to_mel(f):
    """Slaney mel scale: linear (f / (200/3)) below 1 kHz, logarithmic above."""
    f = np.asarray(f, dtype=np.float64)
    lin = f / _F_SP
    with np.errstate(divide="ignore"):
        log = _MIN_LOG_MEL + np.log(np.maximum(f, 1e-300) / _MIN_LOG_HZ) / _LOGSTEP
    return np.where(f >= _MIN_LOG_HZ, log, lin)


def mel_to_hz(m):
    m = np.asarray(m, dtype=np.float64)
    return np.where(m >= _MIN_LOG_MEL, _MIN_LOG_HZ * np.exp(_LOGSTEP * (m - _MIN_LOG_MEL)), _F_SP * m)


def mel_filterbank(n_mels: int = 128, n_freqs: int = N_FFT // 2 + 1, sample_rate: int = SAMPLE_RATE) -> np.ndarray:
    """[n_freqs, n_mels] slaney filterbank (triangles between n_mels + 2 points equally spaced
    on the mel scale from 0 to sample_rate / 2, each scaled by 2 / (its bandwidth in Hz))."""
    all_freqs = np.linspace(0.0, sample_rate // 2, n_freqs)
    m_pts = np.linspace(hz_to_mel(0.0), hz_to_mel(float(sample_rate // 2)), n_mels + 2)
    f_pts = mel_to_hz(m_pts)
    f_diff = f_pts[1:] - f_pts[:-1]
    slopes = f_pts[None, :] - all_freqs[:, None]
    down = -slopes[:, :-2] / f_diff[:-1]
    up = slopes[:, 2:] / f_diff[1:]
    fb = np.maximum(0.0, np.minimum(down, up))
    return fb * (2.0 / (f_pts[2 : n_mels + 2] - f_pts[:n_mels]))[None, :]


def power_spectrum(waveform) -> np.ndarray:
    """|STFT|^2 of every frame but the last: [201, n_samples // 160] (audio.py:143-150)."""
    x = np.asarray(waveform, dtype=np.float64)
    xp = np.pad(x, (N_FFT // 2, N_FFT // 2), mode="reflect")
    n_frames = 1 + (xp.shape[0] - N_FFT) // HOP_LENGTH
    idx = np.arange(N_FFT)[None, :] + HOP_LENGTH * np.arange(n_frames)[:, None]
    window = 0.5 - 0.5 * np.cos(2.0 * np.pi * np.arange(N_FFT) / N_FFT)  # periodic Hann
    spec = np.fft.rfft(xp[idx] * window[None, :], axis=-1)  # [frames, 201]
    return (np.abs(spec[:-1]) ** 2).T


def log_mel_ref(waveform, n_mels: int = 128, target_frames: int | None = None) -> np.ndarray:
    """LogMelSpectrogram._process_single_audio (audio.py:128-156) in float64: [n_mels, frames]."""
    mel = mel_filterbank(n_mels).T @ power_spectrum(waveform)
    log_spec = np.log10(np.maximum(mel, 1e-10))
    log_spec = np.maximum(log_spec, log_spec.max() - 8.0)
    out = (log_spec + 4.0) / 4.0
    if target_frames is None:
        return out
    if out.shape[-1] < target_frames:
        return np.pad(out, ((0, 0), (0, target_frames - out.shape[-1])), constant_values=-1.5)
    return out[:, :target_frames]


def log_mel_torch(waveform, fb, target_frames: int | None = None):
    """The reference's op sequence in torch fp32 on the CPU (audio.py:141-156), with the given
    [201, n_mels] filterbank in place of torchaudio's MelScale. The timed CPU baseline."""
    import torch

    w = torch.as_tensor(waveform, dtype=torch.float32)
    stft = torch.stft(w, N_FFT, HOP_LENGTH, window=torch.hann_window(N_FFT), return_complex=True)
    magnitudes = stft[..., :-1].abs() ** 2
    mel = torch.matmul(magnitudes.transpose(-1, -2), torch.as_tensor(fb, dtype=torch.float32)).transpose(-1, -2)
    log_spec = torch.clamp(mel, min=1e-10).log10()
    log_spec = torch.maximum(log_spec, log_spec.max() - 8.0)
    out = (log_spec + 4.0) / 4.0
    if target_frames is not None:
        if out.shape[-1] < target_frames:
            out = torch.nn.functional.pad(out, (0, target_frames - out.shape[-1]), value=-1.5)
        else:
            out = out[..., :target_frames]
    return out
