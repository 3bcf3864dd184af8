"""Host-side logic that needs no GPU: the Python shim's argument handling, the slot cache
(reference model.py:98-192 semantics), the HBM slot planner, and the decoder plumbing run on
the CPU through the oracle's torch attention (the reference's own CPU arithmetic)."""
import numpy as np
import pytest
import torch

from oracle.attention_oracle import kvcache_torch, sdpa_torch


def test_shim_rejects_cpu_tensors_and_unsupported_options():
    from whisperdrz_amd import flash_attn_with_kvcache, scaled_dot_product_attention

    q = torch.randn(1, 2, 4, 64)
    with pytest.raises(RuntimeError, match="GPU only"):
        scaled_dot_product_attention(q, q, q)
    with pytest.raises(NotImplementedError):
        scaled_dot_product_attention(q, q, q, attn_mask=torch.ones(4, 4, dtype=torch.bool))
    with pytest.raises(NotImplementedError):
        scaled_dot_product_attention(q, q, q, dropout_p=0.1)
    with pytest.raises(RuntimeError, match="GPU only"):
        flash_attn_with_kvcache(torch.randn(1, 1, 2, 64), torch.randn(2, 8, 2, 64), torch.randn(2, 8, 2, 64))


def test_product_has_no_oracle_dependency():
    import pathlib
    import re

    pkg = pathlib.Path(__file__).resolve().parents[1] / "whisperdrz_amd"
    for f in pkg.rglob("*.py"):
        assert not re.search(r"^\s*(from|import)\s+oracle", f.read_text(), flags=re.M), f


def test_flash_kv_cache_semantics():
    from whisperdrz_amd.kv_cache import FlashKVCache

    c = FlashKVCache(4, 10, 2, 64, dtype=torch.float32)
    assert c.k_cache.shape == (4, 10, 2, 64) and c.k_storage.shape == (4, 2, 10, 64)
    assert c.k_cache.stride(-1) == 1 and c.k_cache.stride(1) == 64 and c.k_cache.stride(2) == 640
    k = torch.randn(2, 3, 2, 64)
    v = torch.randn(2, 3, 2, 64)
    slots = torch.tensor([3, 1])
    c.prefill(k, v, start_pos=2, slot_indices=slots)
    assert torch.equal(c.k_cache[3, 2:5], k[0]) and torch.equal(c.v_cache[1, 2:5], v[1])
    assert c.seq_lens.tolist() == [0, 5, 0, 5]
    c.prefill(k, v)  # no slots: rows [:B]
    assert c.seq_lens.tolist() == [3, 3, 0, 5]
    x = torch.randn(2, 7, 2, 64)
    c.set_cross_attention(x, x, slot_indices=torch.tensor([0, 2]))
    assert c.done and c.cross_attn_len == 7 and torch.equal(c.k_cache[2, :7], x[1])
    c.reset(torch.tensor([1]))
    assert c.seq_lens.tolist() == [3, 0, 0, 5]
    assert torch.equal(c.k_cache[3, 2:5], k[0])  # K/V are not cleared
    c.reset()
    assert c.seq_lens.tolist() == [0, 0, 0, 0] and not c.done


def test_slot_pool_layout_and_plan():
    from whisperdrz_amd.kv_cache import KVSlotPool, cache_bytes_per_slot, plan_slots

    pool = KVSlotPool(3, 5, n_heads=2, head_dim=64, self_len=12, cross_len=20, dtype=torch.bfloat16)
    assert len(pool.self_kv) == 3 and len(pool.cross_kv) == 3
    for kv in pool.self_kv + pool.cross_kv:
        assert (kv.k_storage.data_ptr() - pool.arena.data_ptr()) % (2 << 20) == 0
        assert kv.k_storage.untyped_storage().data_ptr() == pool.arena.untyped_storage().data_ptr()
    pool.self_kv[1].k_cache[2, 3] = 1.0
    assert float(pool.self_kv[1].k_storage[2, :, 3].float().sum()) == 128.0
    assert float(pool.self_kv[0].k_storage.float().abs().sum()) == 0.0
    # Whisper large-v3 per-slot footprint (32 layers, 448 + 1500 positions, bf16): 319 MB
    per = cache_bytes_per_slot(32, 20, 64, 448, 1500, torch.bfloat16)
    assert per == 32 * 2 * 20 * 64 * 2 * (448 + 1500)
    plan = plan_slots(272 * 10**9)
    assert 840 <= plan.n_slots <= 853 and plan.total_bytes <= 272 * 10**9


def _ref_kvcache(q, k_cache, v_cache, k=None, v=None, cache_seqlens=None, cache_batch_idx=None,
                 softmax_scale=None, causal=False):
    return kvcache_torch(q, k_cache, v_cache, k, v, cache_seqlens, cache_batch_idx, softmax_scale)


def _ref_dense(q, k, v, is_causal=False, scale=None):
    return sdpa_torch(q, k, v, scale=scale, causal=is_causal)


def test_decoder_plumbing_cached_equals_uncached_on_cpu():
    """Prefill + cached single-token steps reproduce the uncached forward (model.py:547-617),
    with the reference's torch arithmetic plugged into both seams."""
    from whisperdrz_amd.decoder import TextDecoderStack
    from whisperdrz_amd.kv_cache import KVSlotPool

    torch.manual_seed(0)
    dec = TextDecoderStack(100, 16, 128, 2, 2, attn_kvcache=_ref_kvcache, attn_dense=_ref_dense).eval()
    pool = KVSlotPool(2, 3, 2, 64, self_len=16, cross_len=10, dtype=torch.float32)
    xa = torch.randn(2, 10, 128)
    toks = torch.randint(0, 100, (2, 7))
    slots = torch.tensor([2, 0])
    with torch.no_grad():
        full = dec(toks, xa)
        outs = [dec.prefill_flash(toks[:, :3], xa, pool.self_kv, pool.cross_kv, slot_indices=slots)]
        for t in range(3, 7):
            pos = pool.self_kv[0].seq_lens[slots].long()
            outs.append(dec.forward_flash(toks[:, t : t + 1], pool.self_kv, pool.cross_kv, pos, slot_indices=slots))
    np.testing.assert_allclose(torch.cat(outs, 1).numpy(), full.numpy(), rtol=1e-4, atol=1e-5)
    assert pool.self_kv[1].seq_lens.tolist() == [7, 0, 7]


def test_graph_bucket_choice():
    from whisperdrz_amd.decoder import GRAPH_BUCKETS, bucket_for

    assert [bucket_for(b, GRAPH_BUCKETS) for b in (1, 3, 9, 33, 53, 54, 60)] == [1, 4, 16, 42, 54, 54, 60]


def test_lengths_matrix_detects_the_pool_layout():
    from whisperdrz_amd.decoder import lengths_matrix
    from whisperdrz_amd.kv_cache import FlashKVCache, KVSlotPool

    pool = KVSlotPool(3, 4, 2, 64, self_len=16, cross_len=8, dtype=torch.float32)
    m = lengths_matrix(pool.self_kv)
    assert m is pool.self_seq_lens and m.shape == (3, 4)
    pool.self_kv[1].seq_lens[2] = 7  # each layer's lengths are its own row
    assert int(m[1, 2]) == 7 and int(m[0, 2]) == 0
    pool.self_kv[0].reset()
    assert int(m[1, 2]) == 7
    separate = [FlashKVCache(4, 16, 2, 64, dtype=torch.float32) for _ in range(3)]
    assert lengths_matrix(separate) is None
    assert lengths_matrix([pool.self_kv[0], pool.self_kv[2]]) is None  # not the rows in order


def test_fused_projection_weights_track_the_parameters():
    from whisperdrz_amd.decoder import MultiHeadAttention

    torch.manual_seed(0)
    m = MultiHeadAttention(64, 2)
    w, b = m.qkv_weight()
    assert torch.equal(w, torch.cat([m.query.weight, m.key.weight, m.value.weight]))
    assert torch.equal(b[64:128], torch.zeros(64)) and torch.equal(b[128:], m.value.bias)
    assert m.qkv_weight()[0] is w  # cached
    with torch.no_grad():
        m.value.weight.mul_(2)  # an in-place change rebuilds it
    w2, _ = m.qkv_weight()
    assert w2 is not w and torch.equal(w2[128:], m.value.weight)
    kw, kb = m.kv_weight()
    assert torch.equal(kw, torch.cat([m.key.weight, m.value.weight])) and torch.equal(kb[:64], torch.zeros(64))
    x = torch.randn(3, 5, 64)
    qkv = torch.nn.functional.linear(x, *m.qkv_weight())
    torch.testing.assert_close(qkv[..., 64:128], m.key(x))
    torch.testing.assert_close(qkv[..., 128:], m.value(x))


def test_cpu_cache_writes_keep_torch_indexing():
    # the HIP fill takes GPU tensors only; CPU caches are written by torch indexing as before
    from whisperdrz_amd.kv_cache import FlashKVCache

    c = FlashKVCache(4, 10, 2, 64, dtype=torch.float32)
    k, v = torch.randn(2, 3, 2, 64), torch.randn(2, 3, 2, 64)
    c.prefill(k, v, 5, torch.tensor([3, 1]))
    assert torch.equal(c.k_cache[3, 5:8], k[0]) and torch.equal(c.v_cache[1, 5:8], v[1])
    assert c.seq_lens.tolist() == [0, 8, 0, 8]
    c.set_cross_attention(k, v, torch.tensor([0, 2]))
    assert torch.equal(c.k_cache[2, :3], k[1]) and c.cross_attn_len == 3
