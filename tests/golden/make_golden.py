"""Writes the golden fixtures in this folder: small seeded inputs and float64 expected outputs.

Expected outputs come from the CPU oracle (oracle/attention_oracle.py, itself pinned by
tests/test_oracle.py) and are cross-checked here against torch's CPU SDPA / the torch
restatement of the reference fallback before being written. 16-bit cases store the already
rounded inputs (as float32) so the expectation is exact for the values the kernel sees.

Run: python tests/golden/make_golden.py   (deterministic; rewrites the .npz files)
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle.attention_oracle import kvcache_ref, kvcache_torch, sdpa_ref, sdpa_torch  # noqa: E402


def rounded(x, dtype):
    return torch.from_numpy(x.astype(np.float32)).to(dtype).to(torch.float32).numpy()


def dense_case(name, B, H, Lq, Lk, causal, dtype, seed):
    r = np.random.default_rng(seed)
    q, k, v = (rounded(r.standard_normal((B, H, L, 64)), dtype) for L in (Lq, Lk, Lk))
    out = sdpa_ref(q, k, v, scale=0.125, causal=causal)
    chk = sdpa_torch(*(torch.from_numpy(x.astype(np.float64)) for x in (q, k, v)), scale=0.125, causal=causal)
    assert np.max(np.abs(chk.numpy() - out)) < 1e-10
    np.savez_compressed(os.path.join(HERE, f"dense_{name}.npz"), q=q, k=k, v=v, out=out,
                        causal=np.array(causal), dtype=np.array(str(dtype).split(".")[1]))


def kv_case(name, B, sq, H, S, Lmax, self_attn, dtype, seed):
    r = np.random.default_rng(seed)
    q = rounded(r.standard_normal((B, sq, H, 64)), dtype)
    kc = rounded(r.standard_normal((S, Lmax, H, 64)), dtype)
    vc = rounded(r.standard_normal((S, Lmax, H, 64)), dtype)
    idx = r.permutation(S)[:B].astype(np.int32)
    if self_attn:
        kn = rounded(r.standard_normal((B, sq, H, 64)), dtype)
        vn = rounded(r.standard_normal((B, sq, H, 64)), dtype)
        cs = r.integers(0, Lmax - sq + 1, size=B).astype(np.int32)
        cs[0] = 0
        out, k2, v2 = kvcache_ref(q, kc, vc, kn, vn, cs, idx, 0.125)
        T = lambda x: torch.from_numpy(np.array(x, dtype=np.float64))
        chk = kvcache_torch(T(q), T(kc), T(vc), T(kn), T(vn), torch.from_numpy(cs), torch.from_numpy(idx), 0.125)
    else:
        kn = vn = np.zeros((0,), np.float32)
        cs = np.zeros((0,), np.int32)
        out, k2, v2 = kvcache_ref(q, kc, vc, cache_batch_idx=idx, softmax_scale=0.125)
        T = lambda x: torch.from_numpy(np.array(x, dtype=np.float64))
        chk = kvcache_torch(T(q), T(kc), T(vc), cache_batch_idx=torch.from_numpy(idx), softmax_scale=0.125)
    assert np.max(np.abs(chk.numpy() - out)) < 1e-10
    np.savez_compressed(os.path.join(HERE, f"kv_{name}.npz"), q=q, k_cache=kc, v_cache=vc, k=kn, v=vn,
                        cache_seqlens=cs, cache_batch_idx=idx, out=out, k_cache_after=k2, v_cache_after=v2,
                        self_attn=np.array(self_attn), dtype=np.array(str(dtype).split(".")[1]))


def main():
    dense_case("bf16_noncausal", 1, 2, 45, 70, False, torch.bfloat16, 1)
    dense_case("bf16_causal", 1, 2, 67, 67, True, torch.bfloat16, 2)
    dense_case("fp32_noncausal", 1, 2, 33, 90, False, torch.float32, 3)
    kv_case("bf16_self_sq1", 3, 1, 2, 5, 40, True, torch.bfloat16, 4)
    kv_case("bf16_self_sq5", 3, 5, 2, 5, 40, True, torch.bfloat16, 5)
    kv_case("fp32_self_sq1", 2, 1, 2, 4, 33, True, torch.float32, 6)
    kv_case("bf16_cross_sq1", 3, 1, 2, 4, 50, False, torch.bfloat16, 7)


if __name__ == "__main__":
    main()
