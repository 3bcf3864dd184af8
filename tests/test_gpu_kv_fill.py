"""GPU parity of the cache writes (wdrz_kv_fill via FlashKVCache.prefill / set_cross_attention)
against torch's index_put on the same views (the reference's FlashKVCache, model.py:150-183):
bit-exact, every element of both caches compared (rows outside the written range untouched)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

H, D = 20, 64


def _cache(cuda, dtype, n_slots, Lmax, seed):
    from whisperdrz_amd.kv_cache import FlashKVCache

    g = torch.Generator(device=cuda).manual_seed(seed)
    c = FlashKVCache(n_slots, Lmax, H, D, dtype=dtype, device=cuda)
    c.k_storage.copy_(torch.randn(c.k_storage.shape, generator=g, device=cuda).to(dtype))
    c.v_storage.copy_(torch.randn(c.v_storage.shape, generator=g, device=cuda).to(dtype))
    return c


def _ref_write(c, k, v, slots, start):
    kc, vc = c.k_cache.clone(), c.v_cache.clone()
    T = k.shape[1]
    if slots is None:
        kc[: k.shape[0], start : start + T] = k
        vc[: k.shape[0], start : start + T] = v
    else:
        kc[slots, start : start + T] = k
        vc[slots, start : start + T] = v
    return kc, vc


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,n_slots,Lmax,start,slots", [
    (3, 1500, 5, 1500, 0, [4, 0, 2]),      # cross fill into scattered slots
    (4, 7, 6, 448, 0, None),               # prompt prefill, identity slots
    (2, 5, 3, 448, 443, [1, 2]),           # rows ending at the cache end
    (1, 33, 2, 64, 9, [1]),                # T not a multiple of the 32-row block
])
def test_prefill_matches_index_put(cuda, dtype, B, T, n_slots, Lmax, start, slots):
    c = _cache(cuda, dtype, n_slots, Lmax, seed=B + T)
    g = torch.Generator(device=cuda).manual_seed(7 + T)
    kv = torch.randn((B, T, 2, H, D), generator=g, device=cuda).to(dtype)  # one fused projection
    k, v = kv[:, :, 0], kv[:, :, 1]
    sl = None if slots is None else torch.tensor(slots, device=cuda)
    want_k, want_v = _ref_write(c, k, v, sl, start)
    print(f"kv_fill {dtype} B={B} T={T} start={start} slots={slots}", flush=True)
    c.prefill(k, v, start, sl)
    torch.cuda.synchronize()
    assert torch.equal(c.k_cache, want_k) and torch.equal(c.v_cache, want_v)
    if sl is not None:
        assert c.seq_lens[sl].tolist() == [start + T] * B


def test_cross_attention_fill_and_invalid_slots(cuda):
    c = _cache(cuda, torch.bfloat16, 4, 300, seed=1)
    g = torch.Generator(device=cuda).manual_seed(2)
    k = torch.randn((3, 300, H, D), generator=g, device=cuda).to(torch.bfloat16)
    v = torch.randn((3, 300, H, D), generator=g, device=cuda).to(torch.bfloat16)
    before_k, before_v = c.k_cache.clone(), c.v_cache.clone()
    sl = torch.tensor([2, 7, 0], device=cuda)  # slot 7 does not exist: its row is skipped
    print("kv_fill cross + invalid slot", flush=True)
    c.set_cross_attention(k, v, sl)
    torch.cuda.synchronize()
    assert torch.equal(c.k_cache[2], k[0]) and torch.equal(c.v_cache[0], v[2])
    assert torch.equal(c.k_cache[1], before_k[1]) and torch.equal(c.v_cache[3], before_v[3])
    assert c.cross_attn_len == 300 and c.done


def test_pool_cross_fill_through_prefill_flash(cuda):
    # the decoder's fused key/value projection written by wdrz_kv_fill equals the separate
    # projections written by index_put
    from whisperdrz_amd.decoder import TextDecoderStack
    from whisperdrz_amd.kv_cache import KVSlotPool

    torch.manual_seed(0)
    dec = TextDecoderStack(256, 32, 128, 2, 2).to(cuda, torch.bfloat16).eval()
    pool = KVSlotPool(2, 4, 2, 64, self_len=32, cross_len=50, dtype=torch.bfloat16, device=cuda)
    xa = torch.randn(2, 50, 128, device=cuda).to(torch.bfloat16)
    slots = torch.tensor([3, 1], device=cuda)
    tokens = torch.randint(0, 256, (2, 3), device=cuda)
    print("kv_fill through prefill_flash", flush=True)
    with torch.no_grad():
        dec.prefill_flash(tokens, xa, pool.self_kv, pool.cross_kv, slot_indices=slots)
        for blk, c in zip(dec.blocks, pool.cross_kv):
            k = blk.cross_attn.key(xa).view(2, 50, 2, 64)
            v = blk.cross_attn.value(xa).view(2, 50, 2, 64)
            torch.testing.assert_close(c.k_cache[slots], k, rtol=0, atol=0)
            torch.testing.assert_close(c.v_cache[slots], v, rtol=0, atol=0)
