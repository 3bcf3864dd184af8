"""Pins the CPU oracle (oracle/attention_oracle.py) before it is trusted as the checker.

The reference ships no tests or golden vectors for this path and its flash-attn dependency is
absent, so every check here comes from facts the mathematics fixes, each chosen so that a
plausible slip (dropped scale, wrong mask alignment, transposed operand, append at the wrong
row, wrong slot mapping) fails at least one of them:
  * closed form for two keys, and explicit Python loops on tiny inputs;
  * a single key returns its value row; constant keys return the mean of the values;
  * permutation of key rows leaves non-causal outputs unchanged (and changes causal ones);
  * an sq-token causal query equals sq sequential 1-token steps;
  * rows past cache_seqlens + sq and slots not named by cache_batch_idx do not influence the
    result and are not written;
  * the numpy float64 and torch restatements agree (they share no code);
  * batch rows naming the same slot (bucket padding): every cache position holds the new row of
    the LAST batch row covering it, built here position by position, and every row attends over
    that final cache.
"""
import math

import numpy as np
import pytest
import torch

from oracle.attention_oracle import decode_lengths, kvcache_ref, kvcache_torch, sdpa_ref, sdpa_torch

rng = np.random.default_rng(12345)


def test_sdpa_two_keys_closed_form():
    q = rng.standard_normal((1, 1, 1, 4))
    k = rng.standard_normal((1, 1, 2, 4))
    v = rng.standard_normal((1, 1, 2, 4))
    s0, s1 = (q[0, 0, 0] @ k[0, 0, 0]) * 0.5, (q[0, 0, 0] @ k[0, 0, 1]) * 0.5
    w1 = 1.0 / (1.0 + math.exp(s0 - s1))
    expect = (1 - w1) * v[0, 0, 0] + w1 * v[0, 0, 1]
    np.testing.assert_allclose(sdpa_ref(q, k, v, scale=0.5)[0, 0, 0], expect, rtol=1e-12)


def _loops_sdpa(q, k, v, scale, causal):
    B, H, Lq, D = q.shape
    Lk = k.shape[2]
    out = np.zeros_like(q)
    for b in range(B):
        for h in range(H):
            for i in range(Lq):
                w = []
                for j in range(Lk):
                    if causal and j > i:
                        continue
                    w.append((j, math.exp(sum(q[b, h, i, d] * k[b, h, j, d] for d in range(D)) * scale)))
                tot = sum(x for _, x in w)
                for j, x in w:
                    out[b, h, i] += x / tot * v[b, h, j]
    return out


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Lq,Lk", [(3, 3), (2, 5), (5, 2)])
def test_sdpa_matches_explicit_loops(causal, Lq, Lk):
    q = rng.standard_normal((2, 2, Lq, 3))
    k = rng.standard_normal((2, 2, Lk, 3))
    v = rng.standard_normal((2, 2, Lk, 3))
    np.testing.assert_allclose(sdpa_ref(q, k, v, scale=0.7, causal=causal), _loops_sdpa(q, k, v, 0.7, causal),
                               rtol=1e-10, atol=1e-12)


def test_sdpa_single_key_and_constant_keys():
    q = rng.standard_normal((1, 2, 4, 8))
    v = rng.standard_normal((1, 2, 1, 8))
    k = rng.standard_normal((1, 2, 1, 8))
    np.testing.assert_allclose(sdpa_ref(q, k, v), np.broadcast_to(v, q.shape), rtol=1e-12)
    kc = np.broadcast_to(rng.standard_normal((1, 2, 1, 8)), (1, 2, 6, 8))
    vv = rng.standard_normal((1, 2, 6, 8))
    np.testing.assert_allclose(sdpa_ref(q, kc, vv), np.broadcast_to(vv.mean(axis=2, keepdims=True), q.shape),
                               rtol=1e-10)


def test_sdpa_default_scale_is_inverse_sqrt_d():
    q, k, v = (rng.standard_normal((1, 1, 3, 16)) for _ in range(3))
    np.testing.assert_allclose(sdpa_ref(q, k, v), sdpa_ref(q, k, v, scale=0.25), rtol=1e-12)


def test_sdpa_key_permutation():
    q = rng.standard_normal((1, 1, 6, 8))
    k = rng.standard_normal((1, 1, 6, 8))
    v = rng.standard_normal((1, 1, 6, 8))
    p = rng.permutation(6)
    np.testing.assert_allclose(sdpa_ref(q, k[:, :, p], v[:, :, p]), sdpa_ref(q, k, v), rtol=1e-10)
    assert not np.allclose(sdpa_ref(q, k[:, :, p], v[:, :, p], causal=True), sdpa_ref(q, k, v, causal=True))


@pytest.mark.parametrize("causal", [False, True])
def test_numpy_and_torch_sdpa_agree(causal):
    q, k, v = (rng.standard_normal((2, 3, 17, 64)) for _ in range(3))
    t = sdpa_torch(*(torch.from_numpy(x) for x in (q, k, v)), scale=0.125, causal=causal).numpy()
    np.testing.assert_allclose(sdpa_ref(q, k, v, scale=0.125, causal=causal), t, rtol=1e-9, atol=1e-12)


def _kv_case(B=3, sq=2, H=2, S=5, Lmax=12, D=8, seed=0):
    r = np.random.default_rng(seed)
    q = r.standard_normal((B, sq, H, D))
    kc = r.standard_normal((S, Lmax, H, D))
    vc = r.standard_normal((S, Lmax, H, D))
    kn = r.standard_normal((B, sq, H, D))
    vn = r.standard_normal((B, sq, H, D))
    cs = r.integers(0, Lmax - sq + 1, size=B)
    idx = r.permutation(S)[:B]
    return q, kc, vc, kn, vn, cs, idx


def test_kvcache_self_by_hand():
    q, kc, vc, kn, vn, cs, idx = _kv_case()
    out, k2, v2 = kvcache_ref(q, kc, vc, kn, vn, cs, idx, 0.3)
    B, sq, H, D = q.shape
    for b in range(B):
        s, c = idx[b], cs[b]
        np.testing.assert_array_equal(k2[s, c : c + sq], kn[b])
        for t in range(sq):
            keys = np.concatenate([kc[s, :c], kn[b, : t + 1]])
            vals = np.concatenate([vc[s, :c], vn[b, : t + 1]])
            for h in range(H):
                w = np.exp(keys[:, h] @ q[b, t, h] * 0.3)
                np.testing.assert_allclose(out[b, t, h], (w[:, None] * vals[:, h]).sum(0) / w.sum(), rtol=1e-10)


def test_kvcache_untouched_rows_and_slots():
    q, kc, vc, kn, vn, cs, idx = _kv_case(seed=1)
    out, k2, v2 = kvcache_ref(q, kc, vc, kn, vn, cs, idx, 0.3)
    B, sq = q.shape[:2]
    written = np.zeros(kc.shape[:2], dtype=bool)
    for b in range(B):
        written[idx[b], cs[b] : cs[b] + sq] = True
    np.testing.assert_array_equal(k2[~written], kc[~written])
    np.testing.assert_array_equal(v2[~written], vc[~written])
    # garbage beyond each row's range and in unnamed slots does not change the output
    kg, vg = kc.copy(), vc.copy()
    for s in range(kc.shape[0]):
        lim = max([cs[b] + sq for b in range(B) if idx[b] == s], default=0)
        kg[s, lim:] = 1e3
        vg[s, lim:] = -1e3
    out2, _, _ = kvcache_ref(q, kg, vg, kn, vn, cs, idx, 0.3)
    np.testing.assert_allclose(out2, out, rtol=1e-12)


def test_kvcache_multitoken_equals_sequential():
    q, kc, vc, kn, vn, cs, idx = _kv_case(sq=5, Lmax=20, seed=2)
    out, kfin, _ = kvcache_ref(q, kc, vc, kn, vn, cs, idx, 0.3)
    k_cur, v_cur = kc, vc
    steps = []
    for t in range(5):
        o, k_cur, v_cur = kvcache_ref(q[:, t : t + 1], k_cur, v_cur, kn[:, t : t + 1], vn[:, t : t + 1], cs + t, idx, 0.3)
        steps.append(o)
    np.testing.assert_allclose(np.concatenate(steps, axis=1), out, rtol=1e-10)
    np.testing.assert_array_equal(k_cur, kfin)


def test_kvcache_cross_single_and_constant_keys():
    r = np.random.default_rng(3)
    q = r.standard_normal((2, 3, 2, 8))
    vc = r.standard_normal((4, 1, 2, 8))
    kc = r.standard_normal((4, 1, 2, 8))
    out, _, _ = kvcache_ref(q, kc, vc, cache_batch_idx=np.array([3, 1]))
    np.testing.assert_allclose(out, np.broadcast_to(vc[[3, 1]], out.shape), rtol=1e-12)
    kc = np.broadcast_to(r.standard_normal((4, 1, 2, 8)), (4, 7, 2, 8))
    vc = r.standard_normal((4, 7, 2, 8))
    out, _, _ = kvcache_ref(q, kc, vc, cache_batch_idx=np.array([0, 2]))
    expect = vc[[0, 2]].mean(axis=1, keepdims=True)
    np.testing.assert_allclose(out, np.broadcast_to(expect, out.shape), rtol=1e-10)


def test_kvcache_numpy_and_torch_agree():
    q, kc, vc, kn, vn, cs, idx = _kv_case(sq=3, Lmax=16, seed=4)
    out, k2, v2 = kvcache_ref(q, kc, vc, kn, vn, cs, idx, 0.25)
    T = lambda x: torch.from_numpy(np.array(x))
    ktc, vtc = T(kc), T(vc)
    o = kvcache_torch(T(q), ktc, vtc, T(kn), T(vn), T(cs.astype(np.int32)), T(idx.astype(np.int32)), 0.25)
    np.testing.assert_allclose(o.numpy(), out, rtol=1e-9, atol=1e-12)
    np.testing.assert_array_equal(ktc.numpy(), k2)
    oc = kvcache_torch(T(q), T(kc), T(vc), cache_batch_idx=T(idx.astype(np.int32)), softmax_scale=0.25)
    np.testing.assert_allclose(oc.numpy(), kvcache_ref(q, kc, vc, cache_batch_idx=idx, softmax_scale=0.25)[0],
                               rtol=1e-9, atol=1e-12)


def test_decode_lengths_range_and_determinism():
    a = decode_lengths(3, 64, 1, 448)
    assert a.min() >= 1 and a.max() <= 448 and len(a) == 64
    np.testing.assert_array_equal(a, decode_lengths(3, 64, 1, 448))


def _last_writer_cache(kc, kn, cs, idx, sq):
    """The post-append cache built position by position: the highest batch row covering p wins."""
    out = kc.copy()
    S, Lmax = kc.shape[:2]
    for s in range(S):
        for p in range(Lmax):
            cover = [i for i in range(len(idx)) if idx[i] == s and cs[i] <= p < cs[i] + sq]
            if cover:
                w = max(cover)
                out[s, p] = kn[w, p - cs[w]]
    return out


@pytest.mark.parametrize("case", ["identical", "overlap", "disjoint", "three"])
def test_kvcache_duplicate_slots_last_row_wins(case):
    """model.py:49-57 appends row by row before gathering: with repeated slot ids the last row
    covering a position wins, and every row reads the cache after all appends."""
    B, sq, H, S, Lmax, D = 5, 3, 2, 4, 12, 8
    q, kc, vc, kn, vn, _, _ = _kv_case(B=B, sq=sq, H=H, S=S, Lmax=Lmax, D=D, seed=7)
    idx = {"identical": [2, 0, 2, 1, 3], "overlap": [2, 0, 2, 1, 2], "disjoint": [1, 0, 3, 1, 2],
           "three": [3, 3, 0, 3, 1]}[case]
    cs = {"identical": [4, 0, 4, 6, 2], "overlap": [4, 0, 6, 6, 5], "disjoint": [0, 2, 1, 3, 5],
          "three": [2, 3, 0, 4, 8]}[case]
    idx, cs = np.array(idx), np.array(cs)
    out, k2, v2 = kvcache_ref(q, kc, vc, kn, vn, cs, idx, 0.3)
    kf, vf = _last_writer_cache(kc, kn, cs, idx, sq), _last_writer_cache(vc, vn, cs, idx, sq)
    np.testing.assert_array_equal(k2, kf)
    np.testing.assert_array_equal(v2, vf)
    for b in range(B):
        for t in range(sq):
            n = cs[b] + t + 1
            for h in range(H):
                w = np.exp(kf[idx[b], :n, h] @ q[b, t, h] * 0.3)
                np.testing.assert_allclose(out[b, t, h], (w[:, None] * vf[idx[b], :n, h]).sum(0) / w.sum(), rtol=1e-10)
    # the torch restatement follows the same order
    tk, tv = torch.from_numpy(kc.copy()), torch.from_numpy(vc.copy())
    o_t = kvcache_torch(torch.from_numpy(q), tk, tv, torch.from_numpy(kn), torch.from_numpy(vn),
                        torch.from_numpy(cs), torch.from_numpy(idx), 0.3)
    np.testing.assert_array_equal(tk.numpy(), kf)
    np.testing.assert_allclose(o_t.numpy(), out, rtol=1e-9, atol=1e-12)
