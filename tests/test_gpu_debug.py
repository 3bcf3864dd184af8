"""The debug library (WDRZ_DEBUG) rejects bad device metadata on the host before launching,
where the release kernels produce NaN rows (tests/test_gpu_kvcache.py); valid calls give the
release library's results bit for bit."""
import ctypes

import pytest
import torch

from tests._util import make_cache, randn

pytestmark = pytest.mark.gpu
D = 64


@pytest.fixture(scope="module")
def dbg(cuda):
    from whisperdrz_amd import _lib

    lib = ctypes.CDLL(str(_lib.DEBUG_LIB_PATH))
    _lib._declare(lib)
    return lib


def _call(lib, q, kc, vc, k, v, seq, bidx, out):
    from whisperdrz_amd import _lib

    B, sq, H, _ = q.shape
    st = lambda t: (ctypes.c_int64 * 4)(*t.stride())
    return lib.wdrz_attn_kvcache(
        _lib.WDRZ_BF16, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), k.data_ptr(), v.data_ptr(), seq.data_ptr(),
        bidx.data_ptr(), out.data_ptr(), B, sq, H, D, kc.shape[0], kc.shape[1], st(q), st(kc), st(vc), st(k),
        st(v), st(out), ctypes.c_float(0.125), 1, None, 0, torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("case", ["slot", "overflow"])
def test_debug_library_rejects_bad_metadata(cuda, dbg, case):
    from whisperdrz_amd import _lib

    print(f"debug reject: {case}", flush=True)
    kc, vc = make_cache(3, 64, 2, D, torch.bfloat16, cuda, "slot_major", 1)
    snap = kc.clone()
    q = randn((2, 2, 2, D), 2, torch.bfloat16).to(cuda)
    k = randn((2, 2, 2, D), 3, torch.bfloat16).to(cuda)
    bidx, seq = {"slot": ([1, 3], [5, 5]), "overflow": ([1, 0], [5, 63])}[case]
    bidx = torch.tensor(bidx, dtype=torch.int32, device=cuda)
    seq = torch.tensor(seq, dtype=torch.int32, device=cuda)
    out = torch.empty_like(q)
    rc = _call(dbg, q, kc, vc, k, k, seq, bidx, out)
    torch.cuda.synchronize()
    assert rc == _lib.WDRZ_EINVAL
    assert "debug check" in dbg.wdrz_last_error().decode()
    assert torch.equal(kc, snap), "nothing may be launched after a failed check"


def test_debug_library_matches_release_on_valid_calls(cuda, dbg):
    from whisperdrz_amd import _lib

    rel = _lib.load()
    kc, vc = make_cache(4, 448, 20, D, torch.bfloat16, cuda, "head_major", 5)
    kc2, vc2 = kc.clone(), vc.clone()
    q = randn((3, 1, 20, D), 6, torch.bfloat16).to(cuda)
    k = randn((3, 1, 20, D), 7, torch.bfloat16).to(cuda)
    v = randn((3, 1, 20, D), 8, torch.bfloat16).to(cuda)
    # a padded duplicate of row 0 with its own (different) new K/V: row 2 wins the position
    bidx = torch.tensor([2, 0, 2], dtype=torch.int32, device=cuda)
    seq = torch.tensor([100, 7, 100], dtype=torch.int32, device=cuda)
    ws_bytes = rel.wdrz_attn_kvcache_workspace_size(3, 1, 20, D, 448)
    assert ws_bytes > 0
    o1, o2 = torch.empty_like(q), torch.empty_like(q)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=cuda)
    st = lambda t: (ctypes.c_int64 * 4)(*t.stride())
    args = lambda kcx, vcx, o, w: (
        _lib.WDRZ_BF16, q.data_ptr(), kcx.data_ptr(), vcx.data_ptr(), k.data_ptr(), v.data_ptr(), seq.data_ptr(),
        bidx.data_ptr(), o.data_ptr(), 3, 1, 20, D, 4, 448, st(q), st(kcx), st(vcx), st(k), st(v), st(o),
        ctypes.c_float(0.125), 1, w.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    ws2 = torch.zeros_like(ws)
    assert dbg.wdrz_attn_kvcache(*args(kc, vc, o1, ws)) == 0, dbg.wdrz_last_error().decode()
    assert rel.wdrz_attn_kvcache(*args(kc2, vc2, o2, ws2)) == 0, rel.wdrz_last_error().decode()
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(kc, kc2) and torch.equal(vc, vc2)


def test_python_debug_mode_raises(cuda, monkeypatch):
    from whisperdrz_amd import _lib, flash_attn_with_kvcache

    monkeypatch.setattr(_lib, "debug_mode", lambda: True)
    kc, vc = make_cache(3, 64, 2, D, torch.bfloat16, cuda, "slot_major", 1)
    q = randn((2, 1, 2, D), 2, torch.bfloat16).to(cuda)
    with pytest.raises(ValueError, match="slot 3 outside"):
        flash_attn_with_kvcache(q, kc, vc, k=q, v=q, cache_seqlens=torch.tensor([5, 5], dtype=torch.int32, device=cuda),
                                cache_batch_idx=torch.tensor([1, 3], dtype=torch.int32, device=cuda))
