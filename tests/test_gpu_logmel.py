"""GPU parity of the log-mel front end (wdrz_log_mel via whisperdrz_amd.audio) against the
float64 oracle restating LogMelSpectrogram (src/whisperdrz/audio.py:81-156).

Tolerance: 2e-4 max-abs on the scaled log-mel (values in about [-1, 2]); the fp32 DFT's error is
far below the 1e-8 relative power floor the reference applies (max - 8 in log10).
"""
import numpy as np
import pytest
import torch

from oracle.mel_oracle import log_mel_ref

pytestmark = pytest.mark.gpu

TOL = 2e-4


def _noise(n, seed, scale=0.1):
    return (scale * np.random.default_rng(seed).standard_normal(n)).astype(np.float32)


def _tonal(n, seed):
    t = np.arange(n) / 16000.0
    rng = np.random.default_rng(seed)
    x = sum(a * np.sin(2 * np.pi * f * t + rng.uniform(0, 6.28)) for a, f in [(0.3, 220.0), (0.1, 1375.5), (0.05, 5120.0)])
    return (x + 1e-3 * rng.standard_normal(n)).astype(np.float32)


def _check(got, ref, what):
    got = got.detach().cpu().numpy().astype(np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    err = float(np.max(np.abs(got - ref)))
    assert err <= TOL, f"{what}: max|diff|={err:.3e}"


@pytest.mark.parametrize("n_mels", [128, 80])
def test_batch_30s(cuda, n_mels):
    from whisperdrz_amd import log_mel_spectrogram

    x = np.stack([_noise(480000, 1), _tonal(480000, 2)])
    print(f"log-mel B=2 30 s n_mels={n_mels}", flush=True)
    got = log_mel_spectrogram(torch.from_numpy(x).to(cuda), n_mels, target_frames=3000)
    torch.cuda.synchronize()
    for i in range(2):
        _check(got[i], log_mel_ref(x[i], n_mels, 3000), f"window {i}")


@pytest.mark.parametrize("n,target", [(16000 * 7 + 123, None), (160000, 3000), (160000, 500), (201, None), (359, 4)])
def test_lengths_padding_truncation(cuda, n, target):
    from whisperdrz_amd import LogMelSpectrogram

    x = _tonal(n, n)
    print(f"log-mel n={n} target={target}", flush=True)
    got = LogMelSpectrogram(128)(torch.from_numpy(x).to(cuda), target_frames=target)
    torch.cuda.synchronize()
    _check(got, log_mel_ref(x, 128, target), f"n={n} target={target}")


def test_list_and_silence(cuda):
    # the transcriber's call shape: a list of CPU windows of different lengths, padded to 3000
    from whisperdrz_amd import LogMelSpectrogram

    a = _noise(480000, 5)
    a[100000:260000] = 0.0  # 10 s of silence: clamped at 1e-10, floored at max - 8
    b = _tonal(123456, 6)
    print("log-mel list with silence", flush=True)
    got = LogMelSpectrogram(128)([torch.from_numpy(a), torch.from_numpy(b)], target_frames=3000)
    torch.cuda.synchronize()
    assert got.shape == (2, 128, 3000) and got.is_cuda
    _check(got[0], log_mel_ref(a, 128, 3000), "window with silence")
    _check(got[1], log_mel_ref(b, 128, 3000), "short window")
    assert torch.all(got[1, :, 123456 // 160:] == -1.5)


def test_rejects(cuda):
    from whisperdrz_amd import LogMelSpectrogram, log_mel_spectrogram

    with pytest.raises(ValueError):
        log_mel_spectrogram(torch.zeros(200, device=cuda))  # reflect padding needs > 200 samples
    with pytest.raises(NotImplementedError):
        log_mel_spectrogram(torch.zeros(1000, device=cuda), n_mels=129)
    with pytest.raises(NotImplementedError):
        LogMelSpectrogram(128, n_fft=512)
