"""End-to-end plumbing of the decode step (reference model.py:301-362, 570-617, 824-869 and
transcriber.py:31-173): a 2-layer random-weight decoder run with the HIP attention against the
same decoder run with the reference's torch arithmetic (the oracle's restatement of
_sdpa_attn_with_kvcache and SDPA), through prefill, eager decode steps and hipGraph replay.

Tolerance: fp32 logits within 1e-4 * max|ref| (two layers of LayerNorm/MLP amplify the
attention's ~1e-6 relative differences); bf16 and fp16 logits within 2e-2 max-abs relative scale.
"""
import copy

import numpy as np
import pytest
import torch

from oracle.attention_oracle import kvcache_torch, sdpa_torch

pytestmark = pytest.mark.gpu

N_VOCAB, N_CTX, N_STATE, N_HEAD, N_LAYER = 512, 64, 256, 4, 2
CROSS_LEN = 300


def _ref_kvcache(q, k_cache, v_cache, k=None, v=None, cache_seqlens=None, cache_batch_idx=None,
                 softmax_scale=None, causal=False):
    return kvcache_torch(q, k_cache, v_cache, k, v, cache_seqlens, cache_batch_idx, softmax_scale)


def _ref_dense(q, k, v, is_causal=False, scale=None):
    return sdpa_torch(q, k, v, scale=scale, causal=is_causal)


def _make(cuda, dtype, seed=0, n_state=N_STATE, n_head=N_HEAD):
    from whisperdrz_amd.decoder import TextDecoderStack

    torch.manual_seed(seed)
    hip = TextDecoderStack(N_VOCAB, N_CTX, n_state, n_head, N_LAYER).to(cuda, dtype).eval()
    ref = copy.deepcopy(hip)
    ref.fused_small_ops = False  # the reference's separate add and LayerNorm
    for blk in ref.blocks:
        for m in (blk.attn, blk.cross_attn):
            m.attn_kvcache = _ref_kvcache
            m.attn_dense = _ref_dense
    return hip, ref


def _pool(cuda, dtype, n_slots, n_state=N_STATE, n_head=N_HEAD):
    from whisperdrz_amd.kv_cache import KVSlotPool

    return KVSlotPool(N_LAYER, n_slots, n_head, n_state // n_head, self_len=N_CTX, cross_len=CROSS_LEN,
                      dtype=dtype, device=cuda)


def _close(a, b, dtype, what):
    a = a.float().cpu().numpy()
    b = b.float().cpu().numpy()
    scale = float(np.max(np.abs(b)))
    tol = (1e-4 if dtype == torch.float32 else 2e-2) * max(scale, 1.0)
    err = float(np.max(np.abs(a - b)))
    assert np.isfinite(a).all(), what
    assert err <= tol, f"{what}: max|diff|={err:.3e} > {tol:.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_prefill_and_decode_match_reference(cuda, dtype):
    hip, ref = _make(cuda, dtype)
    B, n_slots = 3, 5
    slots = torch.tensor([4, 0, 2], device=cuda)
    g = torch.Generator(device=cuda).manual_seed(1)
    xa = torch.randn(B, CROSS_LEN, N_STATE, generator=g, device=cuda).to(dtype)
    prompt = torch.randint(0, N_VOCAB, (B, 4), generator=g, device=cuda)
    ph, pr = _pool(cuda, dtype, n_slots), _pool(cuda, dtype, n_slots)
    with torch.no_grad():
        lh = hip.prefill_flash(prompt, xa, ph.self_kv, ph.cross_kv, slot_indices=slots)
        lr = ref.prefill_flash(prompt, xa, pr.self_kv, pr.cross_kv, slot_indices=slots)
        _close(lh, lr, dtype, "prefill logits")
        for step in range(6):
            tok = torch.randint(0, N_VOCAB, (B, 1), generator=g, device=cuda)
            pos = ph.self_kv[0].seq_lens[slots].long()
            lh = hip.forward_flash(tok, ph.self_kv, ph.cross_kv, pos, slot_indices=slots)
            lr = ref.forward_flash(tok, pr.self_kv, pr.cross_kv, pos, slot_indices=slots)
            _close(lh, lr, dtype, f"decode step {step}")
        for s_h, s_r in zip(ph.self_kv, pr.self_kv):
            assert torch.equal(s_h.seq_lens, s_r.seq_lens)
            _close(s_h.k_cache, s_r.k_cache, dtype, "self k cache")


def test_uncached_forward_matches_reference(cuda):
    """The DTW-alignment path: causal self SDPA + cross SDPA over the encoder output."""
    hip, ref = _make(cuda, torch.float32, seed=3)
    g = torch.Generator(device=cuda).manual_seed(2)
    xa = torch.randn(2, CROSS_LEN, N_STATE, generator=g, device=cuda)
    toks = torch.randint(0, N_VOCAB, (2, 37), generator=g, device=cuda)
    with torch.no_grad():
        _close(hip(toks, xa), ref(toks, xa), torch.float32, "uncached forward")


def test_cached_decode_equals_uncached_forward(cuda):
    """Prefill + token-by-token cached decode reproduces the uncached full forward."""
    hip, _ = _make(cuda, torch.float32, seed=5)
    B = 2
    g = torch.Generator(device=cuda).manual_seed(4)
    xa = torch.randn(B, CROSS_LEN, N_STATE, generator=g, device=cuda)
    toks = torch.randint(0, N_VOCAB, (B, 9), generator=g, device=cuda)
    pool = _pool(cuda, torch.float32, B)
    with torch.no_grad():
        full = hip(toks, xa)
        steps = [hip.prefill_flash(toks[:, :3], xa, pool.self_kv, pool.cross_kv)]
        for t in range(3, 9):
            pos = pool.self_kv[0].seq_lens.long()
            steps.append(hip.forward_flash(toks[:, t : t + 1], pool.self_kv, pool.cross_kv, pos))
    _close(torch.cat(steps, dim=1), full, torch.float32, "cached vs uncached")


def test_graph_replay_matches_eager(cuda):
    """Captured decode step (hipGraph) replayed several times, with eager work between
    replays, gives the eager results each time."""
    from whisperdrz_amd.decoder import BucketedDecodeGraphs

    dtype = torch.bfloat16
    hip, _ = _make(cuda, dtype, seed=7)
    B = 4
    g = torch.Generator(device=cuda).manual_seed(6)
    xa = torch.randn(B, CROSS_LEN, N_STATE, generator=g, device=cuda).to(dtype)
    prompt = torch.randint(0, N_VOCAB, (B, 3), generator=g, device=cuda)
    slots = torch.arange(B, device=cuda)
    p_graph, p_eager = _pool(cuda, dtype, B), _pool(cuda, dtype, B)
    with torch.no_grad():
        graphs = BucketedDecodeGraphs(hip, p_graph, N_VOCAB, buckets=[4])
        graphs.capture(4)  # warm-up and capture touch slots 0..3; start again from a prefill
        for pool in (p_graph, p_eager):
            pool.reset()
            hip.prefill_flash(prompt, xa, pool.self_kv, pool.cross_kv, slot_indices=slots)
        for step in range(5):
            tok = torch.randint(0, N_VOCAB, (B, 1), generator=g, device=cuda)
            pos = p_eager.self_kv[0].seq_lens.long()
            out_g = graphs.forward(tok, pos, slots).clone()
            torch.cuda.synchronize()
            _ = torch.randn(1000, device=cuda).sum()  # eager work between replays
            out_e = hip.forward_flash(tok, p_eager.self_kv, p_eager.cross_kv, pos, slot_indices=slots)
            torch.cuda.synchronize()
            _close(out_g, out_e, dtype, f"graph replay {step}")
            assert torch.equal(p_graph.self_kv[0].seq_lens, p_eager.self_kv[0].seq_lens)
        assert graphs.hits[4] == 5 and graphs.misses == 0


def test_width_not_multiple_of_128(cuda):
    """A width whose MLP input the fused fc1 + GELU kernel does not take (K % 128 != 0: 320 =
    5 heads x 64) keeps torch's Linear + GELU inside the fused step and still matches."""
    dtype, n_state, n_head = torch.bfloat16, 320, 5
    hip, ref = _make(cuda, dtype, n_state=n_state, n_head=n_head)
    B, n_slots = 2, 3
    slots = torch.tensor([2, 0], device=cuda)
    g = torch.Generator(device=cuda).manual_seed(5)
    xa = torch.randn(B, CROSS_LEN, n_state, generator=g, device=cuda).to(dtype)
    prompt = torch.randint(0, N_VOCAB, (B, 3), generator=g, device=cuda)
    ph, pr = _pool(cuda, dtype, n_slots, n_state, n_head), _pool(cuda, dtype, n_slots, n_state, n_head)
    with torch.no_grad():
        _close(hip.prefill_flash(prompt, xa, ph.self_kv, ph.cross_kv, slot_indices=slots),
               ref.prefill_flash(prompt, xa, pr.self_kv, pr.cross_kv, slot_indices=slots), dtype, "prefill logits")
        for _ in range(3):
            tok = torch.randint(0, N_VOCAB, (B, 1), generator=g, device=cuda)
            pos = ph.self_kv[0].seq_lens[slots].long()
            _close(hip.forward_flash(tok, ph.self_kv, ph.cross_kv, pos, slot_indices=slots),
                   ref.forward_flash(tok, pr.self_kv, pr.cross_kv, pos, slot_indices=slots), dtype, "step logits")
