"""Pins the DTW prep oracle (oracle/dtw_oracle.py) against independent formulations.

The reference ships no tests or fixtures for this path, so the oracle is checked against:
  * scipy.ndimage.median_filter with mode="mirror" (torch's "reflect" padding: the edge sample
    is not repeated) for the median filter, dtw_align.py:65-78;
  * the reference's single-chunk prep, dtw_align.py:772-780 (torch.softmax over the capped
    columns, torch.std_mean(unbiased=False) over all rows, median, mean over heads), which the
    batched prep must equal when every row is valid and the cap is the full width;
  * closed-form invariants: before the filter every column has mean 0 and population std 1
    over the valid rows, masked columns are exactly 0, a 0 cap or 0 length gives NaN, and the
    head mean is linear (the prep of H heads is the mean of the per-head preps with width 1);
  * for compute_attention, the per-head Python loop the reference replaced
    (dtw_align.py:566-585 describe it as the same math).
"""
import numpy as np
import pytest
import scipy.ndimage
import torch

from oracle.dtw_oracle import compute_attention_ref, dtw_prep_ref, dtw_prep_torch, median_filter_ref


@pytest.mark.parametrize("width", [1, 3, 5, 7, 9, 15])
def test_median_filter_matches_scipy_mirror(width):
    rng = np.random.default_rng(width)
    x = rng.standard_normal((3, 4, 41))
    x[0, 0, 5:9] = 0.25  # ties
    got = median_filter_ref(x, width)
    want = scipy.ndimage.median_filter(x, size=(1, 1, width), mode="mirror")
    np.testing.assert_array_equal(got, want)


def test_median_filter_short_axis_is_identity():
    x = np.arange(6.0).reshape(2, 3)
    np.testing.assert_array_equal(median_filter_ref(x, 7), x)  # length 3 <= pad 3
    y = np.array([[3.0, 1.0, 2.0, 0.0]])  # length 4 > pad 3: filtered with reflect padding
    np.testing.assert_array_equal(median_filter_ref(y, 7),
                                  scipy.ndimage.median_filter(y, size=(1, 7), mode="mirror"))


def test_median_filter_torch_reflect_padding():
    # torch's reflect pad, which the reference uses, is numpy's reflect and scipy's mirror
    x = torch.arange(5.0).reshape(1, 1, 5)
    padded = torch.nn.functional.pad(x, (3, 3), mode="reflect").flatten().numpy()
    np.testing.assert_array_equal(padded, np.pad(np.arange(5.0), 3, mode="reflect"))


def _legacy_single_chunk(weights, medfilt_width):
    """dtw_align.py:772-780 for one chunk, full cap, every row valid; then the head mean."""
    w = torch.softmax(torch.as_tensor(weights, dtype=torch.float64), dim=-1)
    std, mean = torch.std_mean(w, dim=-2, keepdim=True, unbiased=False)
    w = ((w - mean) / std).numpy()
    if medfilt_width > 1:
        w = scipy.ndimage.median_filter(w, size=(1, 1, medfilt_width), mode="mirror")
    return w.mean(axis=0)


@pytest.mark.parametrize("width", [1, 7])
def test_prep_equals_reference_single_chunk_path(width):
    rng = np.random.default_rng(7)
    H, T, A = 5, 23, 61
    w = 2.0 * rng.standard_normal((1, H, T, A))
    got = dtw_prep_ref(w, [T], [A], width)[0]
    np.testing.assert_allclose(got, _legacy_single_chunk(w[0], width), rtol=1e-10, atol=1e-10)


def test_prep_cap_equals_truncated_single_chunk_without_filter():
    # with width 1 nothing couples columns, so a cap equals cutting the columns off first
    rng = np.random.default_rng(8)
    H, T, A, cap = 3, 17, 50, 33
    w = 2.0 * rng.standard_normal((1, H, T, A))
    got = dtw_prep_ref(w, [T], [cap], 1)[0]
    np.testing.assert_allclose(got, _legacy_single_chunk(w[0, :, :, :cap], 1), rtol=1e-10, atol=1e-10)


def test_prep_invariants_before_filter():
    rng = np.random.default_rng(9)
    B, T, A = 3, 29, 40
    lens, caps = [29, 11, 20], [40, 25, 7]
    w = 3.0 * rng.standard_normal((B, 1, T, A))
    z = dtw_prep_ref(w, lens, caps, 1)  # H = 1: the head mean is the normalised matrix itself
    assert z.shape == (B, T, max(caps))
    for b in range(B):
        v = z[b, : lens[b], : caps[b]]
        np.testing.assert_allclose(v.mean(axis=0), 0.0, atol=1e-9)
        np.testing.assert_allclose(v.std(axis=0), 1.0, rtol=1e-9)
        assert np.all(z[b, :, caps[b]:] == 0.0)  # masked: p = 0, mean 0, so z = 0 exactly
        # rows past the length are normalised with the same column statistics
        p = np.exp(w[b, 0] - w[b, 0, :, : caps[b]].max(-1, keepdims=True))[:, : caps[b]]
        p /= p.sum(-1, keepdims=True)
        mu, sd = p[: lens[b]].mean(0), p[: lens[b]].std(0)
        np.testing.assert_allclose(z[b, lens[b]:, : caps[b]], ((p - mu) / sd)[lens[b]:], rtol=1e-9, atol=1e-12)


def test_prep_degenerate_rows_are_nan():
    w = np.random.default_rng(1).standard_normal((3, 2, 6, 9))
    z = dtw_prep_ref(w, [6, 0, 4], [9, 5, 0], 3)
    assert np.isfinite(z[0]).all()
    assert np.isnan(z[1]).all() and np.isnan(z[2]).all()


def test_prep_is_mean_of_heads():
    rng = np.random.default_rng(2)
    w = rng.standard_normal((2, 4, 10, 30))
    lens, caps = [10, 6], [30, 21]
    full = dtw_prep_ref(w, lens, caps, 7)
    per_head = np.mean([dtw_prep_ref(w[:, h : h + 1], lens, caps, 7) for h in range(4)], axis=0)
    np.testing.assert_allclose(full, per_head, rtol=1e-12, atol=1e-12)


def test_torch_baseline_matches_oracle():
    rng = np.random.default_rng(3)
    w = (2.0 * rng.standard_normal((2, 3, 12, 40))).astype(np.float32)
    lens, caps = [12, 8], [40, 31]
    np.testing.assert_allclose(dtw_prep_torch(w, lens, caps, 7).numpy(), dtw_prep_ref(w, lens, caps, 7),
                               rtol=1e-4, atol=1e-4)


def test_compute_attention_matches_per_head_loop():
    rng = np.random.default_rng(4)
    n_sel, B, Tt, Ta, D = 3, 2, 5, 7, 64
    q = rng.standard_normal((n_sel, B, Tt, D))
    k = rng.standard_normal((n_sel, B, Ta, D))
    got = compute_attention_ref(q, k, D)
    for i in range(n_sel):
        for b in range(B):
            want = (q[i, b] @ k[i, b].T) / np.sqrt(D)  # (D^-0.25)^2 = D^-0.5
            np.testing.assert_allclose(got[b, i], want, rtol=1e-12)


@pytest.mark.parametrize("width", [1, 3, 7, 15])
def test_median_filter_torch_equals_numpy_restatement(width):
    # the timed torch form and the numpy restatement agree exactly (both select the middle element)
    import torch

    from oracle.dtw_oracle import median_filter_ref, median_filter_torch

    x = np.random.default_rng(width).standard_normal((3, 2, 40)).astype(np.float32)
    got = median_filter_torch(torch.from_numpy(x), width).numpy()
    np.testing.assert_array_equal(got, median_filter_ref(x, width))
    short = x[..., : width // 2]  # no longer than the half width: returned unchanged
    np.testing.assert_array_equal(median_filter_torch(torch.from_numpy(short), width).numpy(), short)
