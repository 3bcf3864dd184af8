"""Parity of the cached decoder kernels at the exact shapes the benchmark times.

Configs 3, 4 and 5 (64 streams, H=20, D=64, head-major slot caches): at this size the launch
walks every row's keys in one workgroup, which small test shapes never reach. Each case runs
one full launch on the GPU and compares every stream with the float64 restatement of
``_sdpa_attn_with_kvcache`` (reference ``src/whisperdrz/model.py:20-76``), computed stream by
stream on the stream's own slot so the host never holds float64 copies of whole caches. The
post-append caches are compared bit for bit with torch's index_put of the new rows.
"""
import numpy as np
import pytest
import torch

from oracle.attention_oracle import decode_lengths, kvcache_ref
from tests._util import TOL_LOWP_ABS

pytestmark = pytest.mark.gpu

B, H, D = 64, 20, 64
LOWP = [torch.bfloat16, torch.float16]


def _cache(n_slots, Lmax, dtype, cuda, seed):
    """Head-major storage [n_slots, H, Lmax, D] handed over as the [n_slots, Lmax, H, D] view."""
    g = torch.Generator(device=cuda).manual_seed(seed)
    kc = torch.randn((n_slots, H, Lmax, D), generator=g, device=cuda, dtype=torch.float32).to(dtype)
    vc = torch.randn((n_slots, H, Lmax, D), generator=g, device=cuda, dtype=torch.float32).to(dtype)
    return kc.permute(0, 2, 1, 3), vc.permute(0, 2, 1, 3)


def _rand(shape, dtype, cuda, seed):
    g = torch.Generator(device=cuda).manual_seed(seed)
    return torch.randn(shape, generator=g, device=cuda, dtype=torch.float32).to(dtype)


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _run(cuda, dtype, sq, Lmax, lengths, seed, check_every=1):
    """One launch at B=64, H=20; returns nothing, asserts parity for every stream (every
    ``check_every``-th stream against the float64 oracle; the caches are compared in full).

    ``lengths`` None: cross-attention over all Lmax rows. Otherwise the attended lengths
    L_i (incl. the sq new tokens), so ``cache_seqlens = L_i - sq``.
    """
    from whisperdrz_amd import flash_attn_with_kvcache, kvcache_workspace_size

    # the benchmark's launch: no key split, no workspace
    assert kvcache_workspace_size(B, sq, H, D, Lmax) == 0, "expected the un-split launch"
    n_slots = B + 16
    rng = np.random.default_rng(seed)
    bidx_np = rng.permutation(n_slots)[:B].astype(np.int32)
    bidx = torch.from_numpy(bidx_np).to(cuda)
    kc, vc = _cache(n_slots, Lmax, dtype, cuda, seed)
    q = _rand((B, sq, H, D), dtype, cuda, seed + 1)
    self_attn = lengths is not None
    if self_attn:
        k = _rand((B, sq, H, D), dtype, cuda, seed + 2)
        v = _rand((B, sq, H, D), dtype, cuda, seed + 3)
        cs_np = (np.asarray(lengths) - sq).astype(np.int32)
        assert cs_np.min() >= 0 and cs_np.max() + sq <= Lmax
        seqlens = torch.from_numpy(cs_np).to(cuda)
        # expected post-append caches (exact copies of the new rows)
        kexp, vexp = kc.clone(), vc.clone()
        for b in range(B):
            s, p = int(bidx_np[b]), int(cs_np[b])
            kexp[s, p : p + sq] = k[b]
            vexp[s, p : p + sq] = v[b]
        # the reference reads the pre-append slot rows
        slot_k = [_np(kc[int(s)]) for s in bidx_np]
        slot_v = [_np(vc[int(s)]) for s in bidx_np]
        out = flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=seqlens, cache_batch_idx=bidx,
                                      softmax_scale=0.125, causal=True)
        torch.cuda.synchronize()
        assert torch.equal(seqlens.cpu(), torch.from_numpy(cs_np)), "cache_seqlens must not change"
        assert torch.equal(kc, kexp), "k_cache differs from the expected post-append cache"
        assert torch.equal(vc, vexp), "v_cache differs from the expected post-append cache"
    else:
        slot_k = [_np(kc[int(s)]) for s in bidx_np]
        slot_v = [_np(vc[int(s)]) for s in bidx_np]
        out = flash_attn_with_kvcache(q, kc, vc, cache_batch_idx=bidx, softmax_scale=0.125)
        torch.cuda.synchronize()
    got = _np(out)
    assert np.isfinite(got).all(), "non-finite output"
    qn = _np(q)
    kn = _np(k) if self_attn else None
    vn = _np(v) if self_attn else None
    worst = 0.0
    for b in range(0, B, check_every):
        if self_attn:
            ref, _, _ = kvcache_ref(qn[b : b + 1], slot_k[b][None], slot_v[b][None], kn[b : b + 1], vn[b : b + 1],
                                    cs_np[b : b + 1], None, 0.125)
        else:
            ref, _, _ = kvcache_ref(qn[b : b + 1], slot_k[b][None], slot_v[b][None], None, None, None, None, 0.125)
        err = float(np.max(np.abs(got[b : b + 1] - ref)))
        worst = max(worst, err)
        assert err <= TOL_LOWP_ABS, f"stream {b} (slot {bidx_np[b]}): max|diff|={err:.3e} > {TOL_LOWP_ABS}"
    print(f"  worst max|diff| over {len(range(0, B, check_every))} streams: {worst:.3e}", flush=True)


@pytest.mark.parametrize("dtype", LOWP)
def test_config3_self_decode(cuda, dtype):
    """Config 3: sq=1, L_i ~ U[1,448] in a 448-row slot (bench seed), plus the extremes."""
    L = decode_lengths(3, B, 1, 448)
    L[0], L[1] = 1, 448
    print(f"config3 self dtype={dtype} sumL={int(L.sum())}", flush=True)
    _run(cuda, dtype, 1, 448, L, seed=31)


@pytest.mark.parametrize("dtype", LOWP)
def test_config4_cross_decode(cuda, dtype):
    """Config 4: sq=1 cross-attention over all 1500 rows."""
    print(f"config4 cross dtype={dtype}", flush=True)
    _run(cuda, dtype, 1, 1500, None, seed=41)


@pytest.mark.parametrize("dtype", LOWP)
def test_config5_verify_self(cuda, dtype):
    """Config 5 self part: a 5-token draft, L_i ~ U[5,448] incl. the draft."""
    L = decode_lengths(5, B, 5, 448)
    L[0], L[1] = 5, 448
    print(f"config5 self dtype={dtype} sumL={int(L.sum())}", flush=True)
    _run(cuda, dtype, 5, 448, L, seed=51)


@pytest.mark.parametrize("dtype", LOWP)
def test_config5_verify_cross(cuda, dtype):
    """Config 5 cross part: 5 queries per stream over all 1500 rows."""
    print(f"config5 cross dtype={dtype}", flush=True)
    _run(cuda, dtype, 5, 1500, None, seed=52)


@pytest.mark.parametrize("dtype", LOWP)
def test_config5_verify_equals_sequential(cuda, dtype):
    """Config 5's check at its full shape: the 5-token draft equals 5 sequential 1-token steps."""
    from whisperdrz_amd import flash_attn_with_kvcache

    sq, Lmax = 5, 448
    L = decode_lengths(5, B, 5, 448)
    cs = torch.from_numpy((L - sq).astype(np.int32)).to(cuda)
    bidx = torch.arange(B, dtype=torch.int32, device=cuda)
    kc, vc = _cache(B, Lmax, dtype, cuda, 53)
    kc2, vc2 = kc.clone(), vc.clone()
    q = _rand((B, sq, H, D), dtype, cuda, 54)
    k = _rand((B, sq, H, D), dtype, cuda, 55)
    v = _rand((B, sq, H, D), dtype, cuda, 56)
    out = flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=cs, cache_batch_idx=bidx, softmax_scale=0.125)
    steps = [
        flash_attn_with_kvcache(q[:, t : t + 1].contiguous(), kc2, vc2, k=k[:, t : t + 1].contiguous(),
                                v=v[:, t : t + 1].contiguous(), cache_seqlens=cs + t, cache_batch_idx=bidx,
                                softmax_scale=0.125)
        for t in range(sq)
    ]
    torch.cuda.synchronize()
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    err = float((out.float() - torch.cat(steps, dim=1).float()).abs().max())
    assert err <= TOL_LOWP_ABS, f"verify vs sequential: {err:.3e}"


@pytest.mark.parametrize("dtype", LOWP)
@pytest.mark.parametrize("sq", [9, 16, 37, 40, 224, 300])
def test_prefill_self(cuda, dtype, sq):
    """Prefill of sq > 8 new tokens into 448-row slots (the prompt of a window): at 64 streams the
    launch takes the multi-query MFMA kernel in 16-row blocks below 40 new rows and the 256-query
    prefill kernel from 40 on (300: two query blocks, the second ragged). Pre-append lengths
    uniform in [0, 448 - sq], with an empty cache and a full one among them."""
    rng = np.random.default_rng(sq)
    L = rng.integers(sq, 448 + 1, size=B)
    L[0], L[1] = sq, 448
    print(f"prefill self dtype={dtype} sq={sq} sumL={int(L.sum())}", flush=True)
    _run(cuda, dtype, sq, 448, L, seed=61 + sq, check_every=4 if sq > 64 else 1)


@pytest.mark.parametrize("dtype", LOWP)
@pytest.mark.parametrize("sq", [24, 64, 224])
def test_prefill_cross(cuda, dtype, sq):
    """sq queries per stream over all 1500 cross rows (a prompt's cross-attention): 16-row blocks
    below 40 queries, the 256-query kernel from 40 on."""
    print(f"prefill cross dtype={dtype} sq={sq}", flush=True)
    _run(cuda, dtype, sq, 1500, None, seed=71 + sq, check_every=4 if sq > 64 else 1)
