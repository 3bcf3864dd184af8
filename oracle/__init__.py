"""CPU oracle for the WhisperDRZ attention hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker / the timed CPU baseline — never as a code path of the
product (``whisperdrz_amd`` does not import it and has no CPU fallback).

Contents (``attention_oracle``):
  * ``sdpa_ref``            — numpy float64 restatement of the dense SDPA call
                              (reference src/whisperdrz/model.py:288-296);
  * ``kvcache_ref``         — numpy float64 restatement of ``_sdpa_attn_with_kvcache``
                              (reference model.py:20-76): sequential in-place append, gather,
                              bottom-right causal mask, SDPA;
  * ``kvcache_torch``       — the same fallback restated with torch on the CPU, the reference's
                              own CPU arithmetic (torch SDPA), used as the timed CPU baseline;
  * ``sdpa_torch``          — torch CPU SDPA (model.py:288-296 exactly as the reference calls it).

Pinning (each function is checked in tests/test_oracle.py against facts fixed by mathematics,
not by re-typing its formula): closed-form two-key softmax; a length-1 key set returns V[0];
constant keys return mean(V); permutation invariance of the non-causal paths; an sq-token
causal query equals sq sequential 1-token steps; rows past ``cache_seqlens + sq`` and slots not
named by ``cache_batch_idx`` are untouched and do not affect the result; and agreement of the
numpy float64 and torch CPU implementations, which share no code. The reference ships no tests
or golden vectors for this path, and flash-attn (un-vendored, version unpinned) is absent, so
its own arithmetic is "parity unpinned"; the fallback's semantics define the contract.
"""
