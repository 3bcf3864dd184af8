"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py): the CPU
oracle still reproduces them (regression guard on the checker itself), and on the GPU the HIP
kernels match them through the C ABI."""
import glob
import os

import numpy as np
import pytest

from oracle.attention_oracle import kvcache_ref, sdpa_ref

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DENSE = sorted(glob.glob(os.path.join(HERE, "dense_*.npz")))
KV = sorted(glob.glob(os.path.join(HERE, "kv_*.npz")))


def test_fixtures_present():
    assert len(DENSE) >= 3 and len(KV) >= 4


@pytest.mark.parametrize("path", DENSE, ids=os.path.basename)
def test_oracle_reproduces_dense_fixture(path):
    f = np.load(path)
    out = sdpa_ref(f["q"], f["k"], f["v"], scale=0.125, causal=bool(f["causal"]))
    np.testing.assert_allclose(out, f["out"], rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("path", KV, ids=os.path.basename)
def test_oracle_reproduces_kv_fixture(path):
    f = np.load(path)
    if bool(f["self_attn"]):
        out, k2, v2 = kvcache_ref(f["q"], f["k_cache"], f["v_cache"], f["k"], f["v"], f["cache_seqlens"],
                                  f["cache_batch_idx"], 0.125)
    else:
        out, k2, v2 = kvcache_ref(f["q"], f["k_cache"], f["v_cache"], cache_batch_idx=f["cache_batch_idx"],
                                  softmax_scale=0.125)
    np.testing.assert_allclose(out, f["out"], rtol=1e-12, atol=1e-14)
    np.testing.assert_array_equal(k2, f["k_cache_after"])
    np.testing.assert_array_equal(v2, f["v_cache_after"])


def _torch_dtype(name):
    import torch

    return {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}[name]


@pytest.mark.gpu
@pytest.mark.parametrize("path", DENSE, ids=os.path.basename)
def test_hip_matches_dense_fixture(cuda, path):
    import torch

    from tests._util import assert_close
    from whisperdrz_amd import scaled_dot_product_attention

    f = np.load(path)
    dt = _torch_dtype(str(f["dtype"]))
    q, k, v = (torch.from_numpy(f[n]).to(dt).to(cuda) for n in ("q", "k", "v"))
    out = scaled_dot_product_attention(q, k, v, is_causal=bool(f["causal"]), scale=0.125)
    torch.cuda.synchronize()
    assert_close(out, f["out"], dt, os.path.basename(path))


@pytest.mark.gpu
@pytest.mark.parametrize("path", KV, ids=os.path.basename)
def test_hip_matches_kv_fixture(cuda, path):
    import torch

    from tests._util import assert_close, to_np
    from whisperdrz_amd import flash_attn_with_kvcache

    f = np.load(path)
    dt = _torch_dtype(str(f["dtype"]))
    T = lambda n: torch.from_numpy(f[n]).to(dt).to(cuda)
    q, kc, vc = T("q"), T("k_cache"), T("v_cache")
    bidx = torch.from_numpy(f["cache_batch_idx"]).to(cuda)
    if bool(f["self_attn"]):
        out = flash_attn_with_kvcache(q, kc, vc, k=T("k"), v=T("v"),
                                      cache_seqlens=torch.from_numpy(f["cache_seqlens"]).to(cuda),
                                      cache_batch_idx=bidx, softmax_scale=0.125)
    else:
        out = flash_attn_with_kvcache(q, kc, vc, cache_batch_idx=bidx, softmax_scale=0.125)
    torch.cuda.synchronize()
    assert_close(out, f["out"], dt, os.path.basename(path))
    assert np.array_equal(to_np(kc), f["k_cache_after"])
    assert np.array_equal(to_np(vc), f["v_cache_after"])
