"""CPU restatement of the reference attention hot path — TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker or the timed CPU baseline. The product (whisperdrz_amd) never imports it.

Citations are to the reference tree (src/whisperdrz/...).
"""
from __future__ import annotations

import numpy as np

# --------------------------------------------------------------------------------------------
# numpy float64 restatements
# --------------------------------------------------------------------------------------------


def _softmax_rows(s: np.ndarray) -> np.ndarray:
    """Row softmax that tolerates fully masked rows being absent (callers never pass one)."""
    m = np.max(s, axis=-1, keepdims=True)
    e = np.exp(s - m)
    return e / np.sum(e, axis=-1, keepdims=True)


def sdpa_ref(q, k, v, scale=None, causal=False) -> np.ndarray:
    """softmax(scale * q k^T [+ top-left causal mask]) v in float64.

    Restates F.scaled_dot_product_attention as called at model.py:288-296 (attn_mask=None,
    dropout 0). q: [B, H, Lq, D], k/v: [B, H, Lk, D]. ``is_causal`` in torch is the top-left
    aligned lower triangle (query i sees keys j <= i). scale None -> D**-0.5 (SDPA default).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    D = q.shape[-1]
    if scale is None:
        scale = D ** -0.5
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    if causal:
        Lq, Lk = s.shape[-2], s.shape[-1]
        mask = np.tril(np.ones((Lq, Lk), dtype=bool))
        s = np.where(mask, s, -np.inf)
    return np.matmul(_softmax_rows(s), v)


def kvcache_ref(
    q,
    k_cache,
    v_cache,
    k=None,
    v=None,
    cache_seqlens=None,
    cache_batch_idx=None,
    softmax_scale=None,
):
    """float64 restatement of _sdpa_attn_with_kvcache (model.py:20-76).

    Returns (out [B, sq, H, D], k_cache', v_cache') where the caches are float64 COPIES with
    the append applied (the reference mutates in place; the copies make the post-append cache
    comparable). Steps, as in the reference:
      1. idx = arange(B) or cache_batch_idx (model.py:40-44);
      2. if k given: for i in range(B): cache[idx[i], cs[i]:cs[i]+sq] = k[i] (49-54);
         keys = cache[idx, :max(cs+sq)]; mask j <= cs[b] + t (55-63);
      3. else keys = cache[idx] (full rows, no mask) (64-67);
      4. SDPA with ``scale=softmax_scale`` over [B, H, sq, *] (69-76).
    """
    q = np.asarray(q, dtype=np.float64)
    kc = np.array(k_cache, dtype=np.float64, copy=True)
    vc = np.array(v_cache, dtype=np.float64, copy=True)
    B, sq, H, D = q.shape
    idx = np.arange(B) if cache_batch_idx is None else np.asarray(cache_batch_idx).astype(np.int64)
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    if k is not None:
        k = np.asarray(k, dtype=np.float64)
        v = np.asarray(v, dtype=np.float64)
        cs = np.asarray(cache_seqlens).astype(np.int64)
        for i in range(B):
            s, p = int(idx[i]), int(cs[i])
            kc[s, p : p + sq] = k[i]
            vc[s, p : p + sq] = v[i]
        max_len = int((cs + sq).max())
        keys = kc[idx, :max_len]
        vals = vc[idx, :max_len]
        jj = np.arange(max_len)
        tt = np.arange(sq)
        mask = jj[None, None, :] <= (cs[:, None, None] + tt[None, :, None])  # [B, sq, max_len]
        mask = mask[:, None]  # [B, 1, sq, max_len]
    else:
        keys = kc[idx]
        vals = vc[idx]
        mask = None
    qh = q.transpose(0, 2, 1, 3)
    kh = keys.transpose(0, 2, 1, 3)
    vh = vals.transpose(0, 2, 1, 3)
    s = np.matmul(qh, np.swapaxes(kh, -1, -2)) * softmax_scale
    if mask is not None:
        s = np.where(mask, s, -np.inf)
    out = np.matmul(_softmax_rows(s), vh)
    return out.transpose(0, 2, 1, 3), kc, vc


# --------------------------------------------------------------------------------------------
# torch CPU restatements (the reference's own CPU arithmetic: torch SDPA)
# --------------------------------------------------------------------------------------------


def sdpa_torch(q, k, v, scale=None, causal=False):
    """torch CPU SDPA exactly as model.py:288-296 calls it (attn_mask None, dropout 0)."""
    import torch.nn.functional as F

    return F.scaled_dot_product_attention(q, k, v, is_causal=causal, attn_mask=None, scale=scale, dropout_p=0.0)


def kvcache_torch(
    q,
    k_cache,
    v_cache,
    k=None,
    v=None,
    cache_seqlens=None,
    cache_batch_idx=None,
    softmax_scale=None,
):
    """torch restatement of _sdpa_attn_with_kvcache (model.py:20-76); mutates the caches."""
    import torch
    import torch.nn.functional as F

    B, sq, _, _ = q.shape
    idx = torch.arange(B, device=q.device) if cache_batch_idx is None else cache_batch_idx.long()
    if k is not None:
        cs = cache_seqlens.long()
        for i in range(B):
            s, p = int(idx[i]), int(cs[i])
            k_cache[s, p : p + sq] = k[i]
            v_cache[s, p : p + sq] = v[i]
        max_len = int((cs + sq).max())
        keys = k_cache[idx, :max_len]
        vals = v_cache[idx, :max_len]
        jj = torch.arange(max_len, device=q.device)
        tt = torch.arange(sq, device=q.device)
        attn_mask = (jj[None, None, :] <= (cs[:, None, None] + tt[None, :, None]))[:, None]
    else:
        keys = k_cache[idx]
        vals = v_cache[idx]
        attn_mask = None
    out = F.scaled_dot_product_attention(
        q.permute(0, 2, 1, 3),
        keys.permute(0, 2, 1, 3),
        vals.permute(0, 2, 1, 3),
        attn_mask=attn_mask,
        scale=softmax_scale,
    )
    return out.permute(0, 2, 1, 3)


# --------------------------------------------------------------------------------------------
# Seeded inputs for the BASELINE configurations (shared by tests and bench)
# --------------------------------------------------------------------------------------------


def decode_lengths(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """Attended lengths L_i ~ U{lo..hi} (inclusive), drawn from the seed."""
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, size=n, dtype=np.int64)
