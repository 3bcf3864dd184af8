"""The allocation-free cached attention entry point (wdrz_attn_kvcache_noalloc) against
wdrz_attn_kvcache with a caller workspace: two calls in a row, the second smaller, both on the
split-KV path that uses the scratch buffer. The two entry points run the same kernels on the
same inputs, so outputs and post-append caches must be bit-identical; the output is also
checked against the float64 restatement of the reference (src/whisperdrz/model.py:20-76)."""
import ctypes

import numpy as np
import pytest
import torch

from oracle.attention_oracle import kvcache_ref
from tests._util import assert_close, make_cache, randn, to_np

pytestmark = pytest.mark.gpu

D = 64


def _strides(t):
    return (ctypes.c_int64 * 4)(*t.stride())


def _call(lib, noalloc, q, kc, vc, k, v, seq, bidx, out, ws):
    from whisperdrz_amd import _lib

    B, sq, H, _ = q.shape
    S, Lmax = kc.shape[0], kc.shape[1]
    stream = torch.cuda.current_stream().cuda_stream
    args = [
        _lib.WDRZ_BF16, q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
        k.data_ptr() if k is not None else None, v.data_ptr() if v is not None else None,
        seq.data_ptr() if seq is not None else None, bidx.data_ptr(), out.data_ptr(),
        B, sq, H, D, S, Lmax,
        _strides(q), _strides(kc), _strides(vc),
        _strides(k if k is not None else q), _strides(v if v is not None else q), _strides(out),
        ctypes.c_float(0.125), 0,
    ]
    if noalloc:
        rc = lib.wdrz_attn_kvcache_noalloc(*args, stream)
    else:
        rc = lib.wdrz_attn_kvcache(*args, ws.data_ptr(), ws.numel(), stream)
    assert rc == 0, lib.wdrz_last_error().decode()


@pytest.mark.parametrize("self_attn", [True, False])
def test_noalloc_matches_workspace_entry(cuda, self_attn):
    from whisperdrz_amd import _lib

    lib = _lib.load()
    # first call larger than the second; both split their keys (workspace > 0)
    shapes = [(3, 5, 20, 1500), (1, 1, 4, 448)]
    for i, (B, sq, H, Lmax) in enumerate(shapes):
        need = lib.wdrz_attn_kvcache_workspace_size(B, sq, H, D, Lmax)
        assert 0 < need <= 4718592, need
        print(f"noalloc call {i}: self={self_attn} B={B} sq={sq} H={H} Lmax={Lmax} workspace={need}", flush=True)
        rng = np.random.default_rng(100 + i)
        n_slots = B + 2
        kc, vc = make_cache(n_slots, Lmax, H, D, torch.bfloat16, cuda, "head_major", 7 + i)
        kc0, vc0 = to_np(kc), to_np(vc)
        kc2, vc2 = kc.clone(), vc.clone()
        q = randn((B, sq, H, D), 20 + i, torch.bfloat16).to(cuda)
        bidx_np = rng.permutation(n_slots)[:B].astype(np.int32)
        bidx = torch.from_numpy(bidx_np).to(cuda)
        if self_attn:
            k = randn((B, sq, H, D), 30 + i, torch.bfloat16).to(cuda)
            v = randn((B, sq, H, D), 40 + i, torch.bfloat16).to(cuda)
            cs = rng.integers(0, Lmax - sq + 1, size=B).astype(np.int32)
            seq = torch.from_numpy(cs).to(cuda)
        else:
            k = v = seq = None
            cs = None
        out_na = torch.empty((B, sq, H, D), dtype=torch.bfloat16, device=cuda)
        out_ws = torch.empty_like(out_na)
        ws = torch.zeros(need, dtype=torch.uint8, device=cuda)
        _call(lib, True, q, kc, vc, k, v, seq, bidx, out_na, None)
        _call(lib, False, q, kc2, vc2, k, v, seq, bidx, out_ws, ws)
        torch.cuda.synchronize()
        assert torch.equal(out_na, out_ws), f"call {i}: no-alloc output differs from the workspace entry point"
        assert torch.equal(kc, kc2) and torch.equal(vc, vc2), f"call {i}: caches differ"
        ref, _, _ = kvcache_ref(to_np(q), kc0, vc0, to_np(k) if self_attn else None,
                                to_np(v) if self_attn else None, cs, bidx_np, 0.125)
        assert_close(out_na, ref, torch.bfloat16, f"no-alloc call {i}")


def test_noalloc_reports_errors(cuda):
    """Bad arguments fail on the host with the library's message, as the workspace entry does."""
    from whisperdrz_amd import _lib

    lib = _lib.load()
    q = torch.zeros((1, 1, 2, D), dtype=torch.bfloat16, device=cuda)
    kc = torch.zeros((2, 64, 2, D), dtype=torch.bfloat16, device=cuda)
    out = torch.empty_like(q)
    st = _strides(q)
    rc = lib.wdrz_attn_kvcache_noalloc(_lib.WDRZ_BF16, q.data_ptr(), kc.data_ptr(), kc.data_ptr(), None, None,
                                       None, None, out.data_ptr(), 1, 1, 2, 32, 2, 64, st, _strides(kc),
                                       _strides(kc), st, st, _strides(out), ctypes.c_float(0.125), 0,
                                       torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.WDRZ_EUNSUPPORTED
    assert "head_dim" in lib.wdrz_last_error().decode()


_CAPTURE_SCRIPT = r"""
import ctypes, sys
import torch
sys.path.insert(0, {root!r})
from whisperdrz_amd import _lib
from tests._util import make_cache, randn
from tests.test_zz_no_alloc import _call

lib = _lib.load()
cuda = torch.device("cuda", 0)
B, sq, H, Lmax, D = 2, 5, 20, 1500, 64
need = lib.wdrz_attn_kvcache_workspace_size(B, sq, H, D, Lmax)
assert need > 0
kc, vc = make_cache(B + 1, Lmax, H, D, torch.bfloat16, cuda, "head_major", 3)
kc2, vc2 = kc.clone(), vc.clone()
q = randn((B, sq, H, D), 4, torch.bfloat16).to(cuda)
k = randn((B, sq, H, D), 5, torch.bfloat16).to(cuda)
v = randn((B, sq, H, D), 6, torch.bfloat16).to(cuda)
seq = torch.tensor([7, 900], dtype=torch.int32, device=cuda)
bidx = torch.tensor([2, 0], dtype=torch.int32, device=cuda)
out_na = torch.zeros((B, sq, H, D), dtype=torch.bfloat16, device=cuda)
out_ws = torch.zeros_like(out_na)
ws = torch.zeros(need, dtype=torch.uint8, device=cuda)
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):  # the process's first no-alloc call: its set-up happens under capture
    _call(lib, True, q, kc, vc, k, v, seq, bidx, out_na, None)
torch.cuda.synchronize()
for rep in range(3):
    out_na.zero_()
    g.replay()
    torch.cuda.synchronize()
    _call(lib, False, q, kc2, vc2, k, v, seq, bidx, out_ws, ws)
    torch.cuda.synchronize()
    assert torch.equal(out_na, out_ws), f"replay {{rep}}: output differs from the workspace entry point"
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2), f"replay {{rep}}: caches differ"
    # an eager no-alloc call between replays shares the scratch array with the graph
    out_e = torch.zeros_like(out_na)
    _call(lib, True, q, kc, vc, k, v, seq, bidx, out_e, None)
    torch.cuda.synchronize()
    assert torch.equal(out_e, out_ws), f"eager call after replay {{rep}} differs"
print("capture-ok")
"""


def test_noalloc_first_call_under_graph_capture(cuda):
    """The first no-alloc call of a process made inside hipGraph capture (its clearing kernel is
    recorded, not run), replayed three times with eager calls between: every replay and every
    eager call bit-identical to the workspace entry point. Runs in a fresh process so that the
    per-device set-up has not happened yet."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("noalloc capture: fresh process", flush=True)
    proc = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT.format(root=root)], cwd=root,
                          capture_output=True, text=True, timeout=110)
    assert proc.returncode == 0 and "capture-ok" in proc.stdout, proc.stdout + proc.stderr
