"""Parity of the cached decoder kernels with the float64 restatement of the reference fallback.

Reference seam: flash_attn_with_kvcache / _sdpa_attn_with_kvcache, src/whisperdrz/model.py:20-95.
"""
import numpy as np
import pytest
import torch

from oracle.attention_oracle import kvcache_ref
from tests._util import assert_close, make_cache, randn, to_np

pytestmark = pytest.mark.gpu

D = 64


def _case(cuda, dtype, B, sq, H, n_slots, Lmax, layout, seed, self_attn=True, bidx_mode="perm", cs=None,
          bidx_np=None):
    from whisperdrz_amd import flash_attn_with_kvcache

    rng = np.random.default_rng(seed)
    kc, vc = make_cache(n_slots, Lmax, H, D, dtype, cuda, layout, seed)
    kc0, vc0 = to_np(kc), to_np(vc)
    q = randn((B, sq, H, D), seed + 10, dtype).to(cuda)
    if bidx_np is not None:
        bidx_np = np.asarray(bidx_np, dtype=np.int32)
        bidx = torch.from_numpy(bidx_np).to(cuda)
    elif bidx_mode == "perm":
        bidx_np = rng.permutation(n_slots)[:B].astype(np.int32)
        bidx = torch.from_numpy(bidx_np).to(cuda)
    else:
        bidx_np, bidx = None, None
    if self_attn:
        k = randn((B, sq, H, D), seed + 11, dtype).to(cuda)
        v = randn((B, sq, H, D), seed + 12, dtype).to(cuda)
        if cs is None:
            cs = rng.integers(0, Lmax - sq + 1, size=B)
            cs[0] = 0
            if B > 1:
                cs[-1] = Lmax - sq
        cs = np.asarray(cs, dtype=np.int32)
        seqlens = torch.from_numpy(cs).to(cuda)
        seqlens_before = seqlens.clone()
        out = flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=seqlens, cache_batch_idx=bidx,
                                      softmax_scale=0.125, causal=True)
        torch.cuda.synchronize()
        assert torch.equal(seqlens, seqlens_before), "cache_seqlens must not be modified"
        ref, kref, vref = kvcache_ref(to_np(q), kc0, vc0, to_np(k), to_np(v), cs, bidx_np, 0.125)
    else:
        out = flash_attn_with_kvcache(q, kc, vc, cache_batch_idx=bidx, softmax_scale=0.125, causal=False)
        torch.cuda.synchronize()
        ref, kref, vref = kvcache_ref(to_np(q), kc0, vc0, None, None, None, bidx_np, 0.125)
    assert out.shape == (B, sq, H, D) and out.dtype == dtype
    assert_close(out, ref, dtype, f"kvcache self={self_attn}")
    # the post-append cache is bit-identical to the reference's (untouched rows/slots included)
    assert np.array_equal(to_np(kc), kref), "k_cache differs from the reference after append"
    assert np.array_equal(to_np(vc), vref), "v_cache differs from the reference after append"
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("sq", [1, 2, 5, 7, 8, 9, 17, 40, 77])
@pytest.mark.parametrize("layout", ["slot_major", "head_major"])
def test_self_attention(cuda, dtype, sq, layout):
    print(f"self dtype={dtype} sq={sq} layout={layout}", flush=True)
    _case(cuda, dtype, B=6, sq=sq, H=4, n_slots=9, Lmax=448, layout=layout, seed=100 + sq)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("Lmax", [1, 63, 100, 1500])
@pytest.mark.parametrize("sq", [1, 5, 45])
def test_cross_attention(cuda, dtype, Lmax, sq):
    print(f"cross dtype={dtype} Lmax={Lmax} sq={sq}", flush=True)
    _case(cuda, dtype, B=5, sq=sq, H=3, n_slots=7, Lmax=Lmax, layout="head_major", seed=200 + Lmax,
          self_attn=False)


@pytest.mark.parametrize("self_attn", [True, False])
def test_identity_batch_idx(cuda, self_attn):
    _case(cuda, torch.bfloat16, B=4, sq=1, H=2, n_slots=4, Lmax=200, layout="slot_major", seed=5,
          self_attn=self_attn, bidx_mode="none")


@pytest.mark.parametrize("B,H,Lmax", [(1, 20, 448), (2, 20, 1500), (1, 1, 1500), (3, 5, 448)])
@pytest.mark.parametrize("self_attn", [True, False])
def test_split_kv_paths(cuda, B, H, Lmax, self_attn):
    """Small batches split the keys over several workgroups (workspace + combine pass)."""
    from whisperdrz_amd import kvcache_workspace_size

    assert kvcache_workspace_size(B, 1, H, D, Lmax) > 0
    _case(cuda, torch.bfloat16, B=B, sq=1, H=H, n_slots=B + 2, Lmax=Lmax, layout="head_major", seed=300 + B,
          self_attn=self_attn)


def _dup_metadata(B, sq, n_slots, Lmax, case, seed):
    """Slot ids with repeats and the lengths the case asks for."""
    rng = np.random.default_rng(seed)
    bidx = rng.permutation(n_slots)[:B].astype(np.int32)
    cs = rng.integers(0, Lmax - sq + 1, size=B).astype(np.int32)
    pairs = [(0, B - 1), (1, B // 2), (2, 3)]
    for j, (src, dst) in enumerate(pairs):
        bidx[dst] = bidx[src]
        if case == "identical":  # bucket padding: a stale slot id with that slot's length
            cs[dst] = cs[src]
        elif case == "overlap":  # regions overlapping by part of the new rows (or shifted by one)
            delta = max(1, sq // 2) * (1 if j % 2 == 0 else -1)
            cs[dst] = cs[src] + delta if 0 <= cs[src] + delta <= Lmax - sq else cs[src] - delta
        else:  # "disjoint": one row appends right behind the other
            cs[dst] = min(Lmax - sq, cs[src] + sq)
    if case == "three":  # three rows on one slot, the middle one appending over both others
        bidx[1] = bidx[2] = bidx[0]
        cs[1] = max(0, cs[0] - 1)
        cs[2] = cs[0]
    return bidx, np.clip(cs, 0, Lmax - sq).astype(np.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("sq", [1, 5, 12, 48])
@pytest.mark.parametrize("B", [6, 64, 70])
@pytest.mark.parametrize("case", ["identical", "overlap", "disjoint", "three"])
def test_duplicate_slots_follow_reference_order(cuda, dtype, sq, B, case):
    """Repeated cache_batch_idx entries (bucket padding, transcriber.py:76-78, 165-167): the
    fallback appends row by row (model.py:51-54), so the last batch row covering a position wins,
    and every row attends over the cache after all appends (model.py:55-57). B=6 takes the
    split-KV path, 64 the one-row-per-workgroup path, 70 the metadata scan beyond one wavefront;
    sq 1 / 5 / 12 / 48 reach kv_attn_kernel, kv_mq_kernel (bf16), the 8-row blocks and
    kv_prefill_kernel (bf16)."""
    if dtype == torch.float32 and sq == 48 and B == 70:
        pytest.skip("fp32 keeps the VALU kernel at every sq; one fp32 case per batch shape is enough")
    print(f"dup case={case} dtype={dtype} sq={sq} B={B}", flush=True)
    n_slots, Lmax, H = B + 4, 448, 3
    bidx, cs = _dup_metadata(B, sq, n_slots, Lmax, case, 1000 + sq + B)
    _case(cuda, dtype, B=B, sq=sq, H=H, n_slots=n_slots, Lmax=Lmax, layout="head_major", seed=700 + sq + B,
          cs=cs, bidx_np=bidx)


def test_config3_shape_fp32_tolerance(cuda):
    """Config 3 shape at fp32: 64 streams, H=20, L_i ~ U[1,448], capacity 448."""
    from oracle.attention_oracle import decode_lengths

    L = decode_lengths(3, 64, 1, 448)
    _case(cuda, torch.float32, B=64, sq=1, H=20, n_slots=64, Lmax=448, layout="head_major", seed=3,
          cs=L - 1)


def test_verify_equals_sequential_steps(cuda):
    """A 5-token causal draft == 5 sequential 1-token steps (config 5's check)."""
    from whisperdrz_amd import flash_attn_with_kvcache

    B, H, Lmax, sq = 8, 20, 448, 5
    for dtype in (torch.bfloat16, torch.float32):
        rng = np.random.default_rng(9)
        cs = rng.integers(0, Lmax - sq + 1, size=B).astype(np.int32)
        kc, vc = make_cache(B, Lmax, H, D, dtype, cuda, "head_major", 9)
        kc2, vc2 = kc.clone(), vc.clone()
        q = randn((B, sq, H, D), 91, dtype).to(cuda)
        k = randn((B, sq, H, D), 92, dtype).to(cuda)
        v = randn((B, sq, H, D), 93, dtype).to(cuda)
        seq = torch.from_numpy(cs).to(cuda)
        bidx = torch.arange(B, dtype=torch.int32, device=cuda)
        out = flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=seq, cache_batch_idx=bidx, softmax_scale=0.125)
        steps = []
        for t in range(sq):
            o = flash_attn_with_kvcache(q[:, t : t + 1].contiguous(), kc2, vc2, k=k[:, t : t + 1].contiguous(),
                                        v=v[:, t : t + 1].contiguous(), cache_seqlens=seq + t, cache_batch_idx=bidx,
                                        softmax_scale=0.125)
            steps.append(o)
        seqout = torch.cat(steps, dim=1)
        torch.cuda.synchronize()
        assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
        assert_close(out, to_np(seqout), dtype, "verify vs sequential")


@pytest.mark.parametrize("sq", [1, 2, 5, 8, 9])
@pytest.mark.parametrize("self_attn", [True, False])
def test_split_workspace_stays_in_bounds(cuda, sq, self_attn):
    """Split-path calls touch exactly the workspace bytes the size query reports: a guard
    region right behind it keeps its bytes, and the workspace itself is left all-zero."""
    from whisperdrz_amd import flash_attn_with_kvcache, kvcache_workspace_size

    B, H, Lmax = 2, 4, 600
    need = kvcache_workspace_size(B, sq, H, D, Lmax)
    assert need > 0, "this shape is meant to take the split path"
    guard = 4096
    buf = torch.zeros(need + guard, dtype=torch.uint8, device=cuda)
    buf[need:] = 0xAB
    rng = np.random.default_rng(sq)
    kc, vc = make_cache(B, Lmax, H, D, torch.bfloat16, cuda, "head_major", 70 + sq)
    kc0, vc0 = to_np(kc), to_np(vc)
    q = randn((B, sq, H, D), 71 + sq, torch.bfloat16).to(cuda)
    bidx_np = np.array([1, 0], dtype=np.int32)
    bidx = torch.from_numpy(bidx_np).to(cuda)
    print(f"workspace guard: sq={sq} self={self_attn} need={need}", flush=True)
    if self_attn:
        k = randn((B, sq, H, D), 72 + sq, torch.bfloat16).to(cuda)
        cs = rng.integers(0, Lmax - sq + 1, size=B).astype(np.int32)
        out = flash_attn_with_kvcache(q, kc, vc, k=k, v=k, cache_seqlens=torch.from_numpy(cs).to(cuda),
                                      cache_batch_idx=bidx, softmax_scale=0.125, workspace=buf[:need])
        ref, _, _ = kvcache_ref(to_np(q), kc0, vc0, to_np(k), to_np(k), cs, bidx_np, 0.125)
    else:
        out = flash_attn_with_kvcache(q, kc, vc, cache_batch_idx=bidx, softmax_scale=0.125, workspace=buf[:need])
        ref, _, _ = kvcache_ref(to_np(q), kc0, vc0, None, None, None, bidx_np, 0.125)
    torch.cuda.synchronize()
    assert_close(out, ref, torch.bfloat16, f"guarded workspace sq={sq}")
    assert int(torch.count_nonzero(buf[:need])) == 0, "workspace not left all-zero"
    assert bool((buf[need:] == 0xAB).all()), "bytes past the reported workspace size were written"


@pytest.mark.parametrize("sq", [1, 4])
@pytest.mark.parametrize("self_attn", [True, False])
def test_bad_slot_gives_nan_not_fault(cuda, sq, self_attn):
    """An out-of-range slot id (which the host cannot see) yields NaN rows and no memory access."""
    from whisperdrz_amd import flash_attn_with_kvcache

    kc, vc = make_cache(3, 64, 2, D, torch.bfloat16, cuda, "slot_major", 1)
    snap_k = kc.clone()
    q = randn((2, sq, 2, D), 2, torch.bfloat16).to(cuda)
    k = randn((2, sq, 2, D), 3, torch.bfloat16).to(cuda)
    bidx = torch.tensor([1, 3], dtype=torch.int32, device=cuda)
    seq = torch.tensor([5, 5], dtype=torch.int32, device=cuda)
    if self_attn:
        out = flash_attn_with_kvcache(q, kc, vc, k=k, v=k, cache_seqlens=seq, cache_batch_idx=bidx)
    else:
        out = flash_attn_with_kvcache(q, kc, vc, cache_batch_idx=bidx)
    torch.cuda.synchronize()
    assert torch.isfinite(out[0].float()).all()
    assert torch.isnan(out[1].float()).all()
    if self_attn:
        snap_k[1, 5 : 5 + sq] = k[0]
    assert torch.equal(kc, snap_k)


def test_prefill_bad_metadata_gives_nan_not_fault(cuda):
    """The prefill kernel (sq >= 40): an out-of-range slot id and a row whose append would run past
    the cache give NaN rows, no append and no memory access; the valid row is appended and finite."""
    from whisperdrz_amd import flash_attn_with_kvcache

    sq, Lmax = 70, 128
    kc, vc = make_cache(3, Lmax, 2, D, torch.bfloat16, cuda, "slot_major", 1)
    snap_k, snap_v = kc.clone(), vc.clone()
    q = randn((3, sq, 2, D), 2, torch.bfloat16).to(cuda)
    k = randn((3, sq, 2, D), 3, torch.bfloat16).to(cuda)
    v = randn((3, sq, 2, D), 4, torch.bfloat16).to(cuda)
    bidx = torch.tensor([1, 3, 2], dtype=torch.int32, device=cuda)   # slot 3 is outside the pool
    seq = torch.tensor([5, 5, 60], dtype=torch.int32, device=cuda)   # 60 + 70 > 128
    out = flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=seq, cache_batch_idx=bidx, causal=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out[0].float()).all()
    assert torch.isnan(out[1].float()).all() and torch.isnan(out[2].float()).all()
    snap_k[1, 5 : 5 + sq] = k[0]
    snap_v[1, 5 : 5 + sq] = v[0]
    assert torch.equal(kc, snap_k) and torch.equal(vc, snap_v)


def test_workspace_reuse_across_shapes(cuda):
    """Split-path calls of different shapes share one workspace; each is correct and the
    workspace is all-zero after every call (its counters start at zero for the next one)."""
    from whisperdrz_amd import flash_attn_with_kvcache, kvcache_workspace_size

    H, Lmax = 6, 700
    shapes = [(1, 1), (3, 5), (2, 1), (1, 9), (4, 2), (1, 1)]
    need = max(kvcache_workspace_size(B, sq, H, D, Lmax) for B, sq in shapes)
    ws = torch.zeros(need, dtype=torch.uint8, device=cuda)
    for i, (B, sq) in enumerate(shapes):
        for self_attn in (True, False):
            print(f"reuse case {i}: B={B} sq={sq} self={self_attn}", flush=True)
            rng = np.random.default_rng(i)
            kc, vc = make_cache(B + 1, Lmax, H, D, torch.bfloat16, cuda, "head_major", 40 + i)
            kc0, vc0 = to_np(kc), to_np(vc)
            q = randn((B, sq, H, D), 50 + i, torch.bfloat16).to(cuda)
            bidx_np = rng.permutation(B + 1)[:B].astype(np.int32)
            bidx = torch.from_numpy(bidx_np).to(cuda)
            if self_attn:
                k = randn((B, sq, H, D), 60 + i, torch.bfloat16).to(cuda)
                cs = rng.integers(0, Lmax - sq + 1, size=B).astype(np.int32)
                out = flash_attn_with_kvcache(q, kc, vc, k=k, v=k, cache_seqlens=torch.from_numpy(cs).to(cuda),
                                              cache_batch_idx=bidx, softmax_scale=0.125, workspace=ws)
                ref, _, _ = kvcache_ref(to_np(q), kc0, vc0, to_np(k), to_np(k), cs, bidx_np, 0.125)
            else:
                out = flash_attn_with_kvcache(q, kc, vc, cache_batch_idx=bidx, softmax_scale=0.125, workspace=ws)
                ref, _, _ = kvcache_ref(to_np(q), kc0, vc0, None, None, None, bidx_np, 0.125)
            torch.cuda.synchronize()
            assert_close(out, ref, torch.bfloat16, f"reuse case {i}")
            assert int(torch.count_nonzero(ws)) == 0, "workspace not left all-zero"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("self_attn", [True, False])
def test_many_rows_need_no_workspace(cuda, dtype, self_attn):
    """sq >= 40 on a small batch (one window's prompt): no workspace is asked for or needed; the
    call through the C ABI with a NULL workspace matches the reference."""
    import ctypes

    from whisperdrz_amd import _lib

    lib = _lib.load()
    B, sq, H, Lmax = 1, 40, 20, 448
    assert lib.wdrz_attn_kvcache_workspace_size(B, sq, H, D, Lmax) == 0
    print(f"no-workspace sq=40 dtype={dtype} self={self_attn}", flush=True)
    kc, vc = make_cache(2, Lmax, H, D, dtype, cuda, "head_major", 41)
    kc0, vc0 = to_np(kc), to_np(vc)
    q = randn((B, sq, H, D), 42, dtype).to(cuda)
    k = randn((B, sq, H, D), 43, dtype).to(cuda) if self_attn else None
    v = randn((B, sq, H, D), 44, dtype).to(cuda) if self_attn else None
    cs = np.array([100], dtype=np.int32)
    seq = torch.from_numpy(cs).to(cuda)
    bidx_np = np.array([1], dtype=np.int32)
    bidx = torch.from_numpy(bidx_np).to(cuda)
    out = torch.empty_like(q)
    st = lambda t: (ctypes.c_int64 * 4)(*t.stride())
    code = {torch.bfloat16: _lib.WDRZ_BF16, torch.float32: _lib.WDRZ_F32}[dtype]
    rc = lib.wdrz_attn_kvcache(code, q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                               k.data_ptr() if self_attn else None, v.data_ptr() if self_attn else None,
                               seq.data_ptr() if self_attn else None, bidx.data_ptr(), out.data_ptr(), B, sq, H, D, 2,
                               Lmax, st(q), st(kc), st(vc), st(k if self_attn else q), st(v if self_attn else q),
                               st(out), ctypes.c_float(0.125), int(self_attn), None, 0,
                               torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.wdrz_last_error().decode()
    torch.cuda.synchronize()
    ref, kref, vref = kvcache_ref(to_np(q), kc0, vc0, to_np(k) if self_attn else None,
                                  to_np(v) if self_attn else None, cs if self_attn else None, bidx_np, 0.125)
    assert_close(out, ref, dtype, "sq=40 without workspace")
    assert np.array_equal(to_np(kc), kref) and np.array_equal(to_np(vc), vref)


@pytest.mark.parametrize("layout", ["head_major", "slot_major"])
def test_prefill_cross_dense_route_slots(cuda, layout):
    """A prompt's cross-attention with enough (row, head) pairs takes the dense hand-scheduled
    kernel through the slot map: a permuted slot map gives the rows of the identity call
    permuted, bit for bit; an out-of-range slot id gives that row NaN and leaves the others
    unchanged; a few rows against the oracle."""
    from whisperdrz_amd import flash_attn_with_kvcache

    B, sq, H, Lmax = 16, 224, 20, 700
    print(f"prefill cross dense route: {layout}", flush=True)
    kc, vc = make_cache(B + 2, Lmax, H, D, torch.bfloat16, cuda, layout, 81)
    q = randn((B, sq, H, D), 82, torch.bfloat16).to(cuda)
    ident = torch.arange(B, dtype=torch.int32, device=cuda)
    perm = torch.from_numpy(np.random.default_rng(83).permutation(B).astype(np.int32)).to(cuda)
    base = flash_attn_with_kvcache(q, kc, vc, cache_batch_idx=ident, softmax_scale=0.125)
    # row i of q against slot perm[i]: equal to the identity call on q with row perm[i]
    qp = torch.empty_like(q)
    qp[torch.arange(B, device=cuda).long()] = q[perm.long()]
    outp = flash_attn_with_kvcache(qp, kc, vc, cache_batch_idx=perm, softmax_scale=0.125)
    bad = perm.clone()
    bad[3] = B + 2  # outside the pool
    outb = flash_attn_with_kvcache(qp, kc, vc, cache_batch_idx=bad, softmax_scale=0.125)
    torch.cuda.synchronize()
    assert torch.equal(outp, base[perm.long()])
    assert torch.isnan(outb[3].float()).all()
    keep = [i for i in range(B) if i != 3]
    assert torch.equal(outb[keep], outp[keep])
    kc_np, vc_np = to_np(kc), to_np(vc)
    for i in (0, 7, B - 1):
        ref = kvcache_ref(to_np(q[i : i + 1]), kc_np, vc_np, None, None, None, np.array([i], np.int32), 0.125)[0]
        assert_close(base[i : i + 1], ref, torch.bfloat16, f"prefill cross row {i}")


@pytest.mark.parametrize("sq", [1, 5, 40])
def test_causal_flag_is_ignored_as_in_the_reference(cuda, sq):
    """The reference fallback (model.py:20-76) never reads `causal`: new rows are always masked
    bottom-right causally and cross calls never are. Same here: causal=False with new rows gives
    the causal result, and causal=True on a cross call changes nothing (bit for bit)."""
    from whisperdrz_amd import flash_attn_with_kvcache

    print(f"causal flag sq={sq}", flush=True)
    B, H, n_slots, Lmax = 4, 3, 6, 448
    q = randn((B, sq, H, D), 900 + sq, torch.bfloat16).to(cuda)
    k = randn((B, sq, H, D), 901 + sq, torch.bfloat16).to(cuda)
    v = randn((B, sq, H, D), 902 + sq, torch.bfloat16).to(cuda)
    bidx = torch.tensor([3, 0, 5, 1], dtype=torch.int32, device=cuda)
    cs = torch.tensor([0, 17, Lmax - sq, 200], dtype=torch.int32, device=cuda)
    outs = {}
    for causal in (True, False):
        kc, vc = make_cache(n_slots, Lmax, H, D, torch.bfloat16, cuda, "head_major", 77)
        outs[causal] = flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=cs, cache_batch_idx=bidx,
                                               softmax_scale=0.125, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(outs[True], outs[False])
    kc, vc = make_cache(n_slots, Lmax, H, D, torch.bfloat16, cuda, "head_major", 77)
    ref, _, _ = kvcache_ref(to_np(q), to_np(kc), to_np(vc), to_np(k), to_np(v), cs.cpu().numpy(), bidx.cpu().numpy(),
                            0.125)
    assert_close(outs[False], ref, torch.bfloat16, "self, causal=False")
    cross = [flash_attn_with_kvcache(q, kc, vc, cache_batch_idx=bidx, softmax_scale=0.125, causal=c)
             for c in (False, True)]
    torch.cuda.synchronize()
    assert torch.equal(cross[0], cross[1])


def test_default_scale_is_head_dim_power(cuda):
    """softmax_scale=None means SDPA's default 1/sqrt(head_dim) (model.py:69-75 passes it to
    F.scaled_dot_product_attention): bit-identical to an explicit 0.125 at head_dim 64."""
    from whisperdrz_amd import flash_attn_with_kvcache, scaled_dot_product_attention

    q = randn((3, 2, 4, D), 31, torch.bfloat16).to(cuda)
    kc, vc = make_cache(5, 300, 4, D, torch.bfloat16, cuda, "head_major", 32)
    bidx = torch.tensor([4, 1, 2], dtype=torch.int32, device=cuda)
    a = flash_attn_with_kvcache(q, kc, vc, cache_batch_idx=bidx)
    b = flash_attn_with_kvcache(q, kc, vc, cache_batch_idx=bidx, softmax_scale=0.125)
    qd = randn((2, 4, 300, D), 33, torch.bfloat16).to(cuda)
    kd = randn((2, 4, 300, D), 34, torch.bfloat16).to(cuda)
    vd = randn((2, 4, 300, D), 35, torch.bfloat16).to(cuda)
    c = scaled_dot_product_attention(qd, kd, vd)
    d = scaled_dot_product_attention(qd, kd, vd, scale=0.125)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(c, d)
