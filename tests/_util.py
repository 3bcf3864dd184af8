"""Helpers shared by the parity tests (tolerances, seeded inputs, cache layouts)."""
from __future__ import annotations

import numpy as np
import torch

# Tolerances from the build's contract: fp32 within 1e-5 relative (max |diff| <= 1e-5 * max |ref|),
# 16-bit types within 2e-2 max-abs of a float reference computed on the same (rounded) inputs.
TOL_F32_REL = 1e-5
TOL_LOWP_ABS = 2e-2


def randn(shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32).to(dtype)


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def assert_close(out: torch.Tensor, ref: np.ndarray, dtype: torch.dtype, what: str = "") -> float:
    got = to_np(out)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = float(np.max(np.abs(got - ref))) if got.size else 0.0
    if dtype == torch.float32:
        bound = TOL_F32_REL * float(np.max(np.abs(ref)))
    else:
        bound = TOL_LOWP_ABS
    assert err <= bound, f"{what}: max|diff|={err:.3e} > {bound:.3e}"
    return err


def make_cache(n_slots, Lmax, H, D, dtype, device, layout, seed):
    """K/V caches viewed as [n_slots, Lmax, H, D].

    layout "slot_major": contiguous [n_slots, Lmax, H, D] (the reference's FlashKVCache layout);
    layout "head_major": storage [n_slots, H, Lmax, D], handed over as a permuted view.
    """
    kc = randn((n_slots, Lmax, H, D), seed, dtype)
    vc = randn((n_slots, Lmax, H, D), seed + 1, dtype)
    if layout == "slot_major":
        return kc.to(device), vc.to(device)
    ks = kc.permute(0, 2, 1, 3).contiguous().to(device)
    vs = vc.permute(0, 2, 1, 3).contiguous().to(device)
    return ks.permute(0, 2, 1, 3), vs.permute(0, 2, 1, 3)
