"""Pins the log-mel oracle (oracle/mel_oracle.py).

The reference ships no tests or fixtures for the front end and its filterbank library
(torchaudio, unpinned) is absent, so:
  * the STFT/power part is checked against torch.stft (center, reflect, periodic Hann), the
    call the reference makes (audio.py:143-150);
  * the slaney mel scale against its closed form: 3 mels per 200 Hz below 1 kHz (15 mels at
    1 kHz), 27 mels per factor 6.4 above, continuous, invertible;
  * the filterbank against what the slaney construction fixes: filter m is a triangle on
    [f_m, f_{m+2}] peaking at f_{m+1} with height 2 / (f_{m+2} - f_m), so its continuous area is
    1 (checked by dense numerical integration of the same breakpoints) — a mel-scale mix-up
    (htk), a missing normalisation or a shifted breakpoint each fail one of these;
  * the log / floor / scale / pad steps against the reference's torch op sequence.
"""
import numpy as np
import pytest
import torch

from oracle.mel_oracle import (
    HOP_LENGTH,
    N_FFT,
    hz_to_mel,
    log_mel_ref,
    log_mel_torch,
    mel_filterbank,
    mel_to_hz,
    power_spectrum,
)


def test_power_spectrum_matches_torch_stft():
    x = np.random.default_rng(0).standard_normal(16000 * 2 + 37)
    st = torch.stft(torch.as_tensor(x), N_FFT, HOP_LENGTH, window=torch.hann_window(N_FFT, dtype=torch.float64),
                    return_complex=True)
    want = (st[..., :-1].abs() ** 2).numpy()
    got = power_spectrum(x)
    assert got.shape == want.shape == (201, (16000 * 2 + 37) // HOP_LENGTH)
    np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-9)


def test_slaney_scale_closed_form():
    assert hz_to_mel(0.0) == 0.0
    np.testing.assert_allclose(hz_to_mel(200.0 / 3.0), 1.0)
    np.testing.assert_allclose(hz_to_mel(1000.0), 15.0)
    np.testing.assert_allclose(hz_to_mel(6400.0), 15.0 + 27.0)  # one factor 6.4 above 1 kHz
    np.testing.assert_allclose(hz_to_mel(999.999999), hz_to_mel(1000.0), atol=1e-6)  # continuous
    f = np.array([0.0, 50.0, 400.0, 999.0, 1000.0, 1500.0, 4000.0, 8000.0])
    np.testing.assert_allclose(mel_to_hz(hz_to_mel(f)), f, rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("n_mels", [80, 128])
def test_filterbank_triangles(n_mels):
    fb = mel_filterbank(n_mels)
    assert fb.shape == (201, n_mels) and (fb >= 0).all()
    f_pts = mel_to_hz(np.linspace(0.0, hz_to_mel(8000.0), n_mels + 2))
    freqs = np.linspace(0.0, 8000.0, 201)
    for m in range(n_mels):
        lo, mid, hi = f_pts[m], f_pts[m + 1], f_pts[m + 2]
        height = 2.0 / (hi - lo)
        col = fb[:, m]
        assert np.all(col[(freqs <= lo) | (freqs >= hi)] == 0.0)
        # linear rise to the peak and fall after it, peak height 2 / bandwidth
        rise = (freqs > lo) & (freqs <= mid)
        fall = (freqs >= mid) & (freqs < hi)
        np.testing.assert_allclose(col[rise], height * (freqs[rise] - lo) / (mid - lo), rtol=1e-12)
        np.testing.assert_allclose(col[fall], height * (hi - freqs[fall]) / (hi - mid), rtol=1e-12)
        # continuous area of that triangle is 1
        dense = np.linspace(lo, hi, 20001)
        tri = height * np.minimum((dense - lo) / (mid - lo), (hi - dense) / (hi - mid))
        np.testing.assert_allclose(np.trapezoid(tri, dense), 1.0, rtol=1e-6)


def test_log_mel_matches_torch_sequence_and_pads():
    x = np.random.default_rng(1).standard_normal(16000 * 3).astype(np.float32)
    fb = mel_filterbank(128)
    ref = log_mel_ref(x)
    got = log_mel_torch(x, fb).numpy()
    assert ref.shape == (128, 300)
    np.testing.assert_allclose(got, ref, atol=2e-5)
    mel = fb.T @ power_spectrum(x)
    assert ref.max() == pytest.approx((np.log10(mel.max()) + 4.0) / 4.0)  # (log10 + 4) / 4
    assert ref.min() >= ref.max() - 2.0 - 1e-12  # floor at max - 8 before the / 4
    quiet = x.copy()
    quiet[16000:32000] = 0.0  # a silent second: clamped at 1e-10, then floored at max - 8
    q = log_mel_ref(quiet)
    np.testing.assert_allclose(q[:, 120:180], q.max() - 2.0)
    padded = log_mel_ref(x, target_frames=320)
    assert padded.shape == (128, 320) and np.all(padded[:, 300:] == -1.5)
    np.testing.assert_array_equal(log_mel_ref(x, target_frames=250), ref[:, :250])
