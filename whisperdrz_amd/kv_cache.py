"""Slot KV caches for the decoder, laid out for one MI355X (288 GB HBM3E).

``FlashKVCache`` keeps the reference's API (``src/whisperdrz/model.py:98-192``): buffers
``k_cache`` / ``v_cache`` indexed ``[slot, pos, head, dim]``, int32 ``seq_lens``, and the
methods ``prefill``, ``set_cross_attention`` and ``reset``. What changes is the storage:

* head-major: each cache is stored as ``[slot, head, pos, dim]`` and exposed as the permuted
  view ``[slot, pos, head, dim]`` that the reference indexes. A (slot, head) pair is then one
  contiguous run of ``pos * 128`` bytes, which is exactly what one attention workgroup streams;
  the attention kernels take strides, so they read the view directly.
* one arena for all layers: ``KVSlotPool`` carves every layer's self and cross caches out of a
  single allocation (2 MiB-aligned slices), so the decoder's 128 cache tensors are one
  allocation whose size is known up front, and ``plan_slots`` sizes the slot count for the
  HBM that is left after weights and activations.

* cache writes on the GPU go through ``wdrz_kv_fill`` (one kernel for K and V, contiguous 4 KB
  runs per (slot, head)) instead of torch's index_put over the permuted view, which is ~3x
  slower on the cross fill.

Sizes at Whisper large-v3 (32 layers, 20 heads, head_dim 64, bf16): 448-position self caches
take 73.4 MB per slot, 1500-position cross caches 245.8 MB per slot, 319 MB per slot in all;
about 850 slots fit in 272 GB.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor

from . import _lib

_ALIGN = 2 << 20  # slice alignment inside the arena (bytes)
_FILL_DTYPES = {torch.bfloat16: _lib.WDRZ_BF16, torch.float16: _lib.WDRZ_F16}


def _hip_fill(k_cache: Tensor, v_cache: Tensor, k: Tensor, v: Tensor, slot_indices: Optional[Tensor],
              start_pos: int) -> bool:
    """``k_cache[slot_indices, start_pos:start_pos + T] = k`` (and v) with ``wdrz_kv_fill``.
    Returns False (nothing written) for what the kernel does not take: CPU tensors, a dtype
    other than the caches' bf16 / fp16, head_dim != 64; the caller then uses torch indexing,
    which also casts."""
    if not (k.is_cuda and k_cache.is_cuda and k.dtype == v.dtype == k_cache.dtype == v_cache.dtype
            and k.dtype in _FILL_DTYPES and k.shape[-1] == 64 and k.dim() == 4):
        return False
    from .attention import _raise, _stream_handle

    B, T, H, D = (int(x) for x in k.shape)
    if tuple(v.shape) != (B, T, H, D) or k_cache.shape[2] != H:
        raise ValueError(f"k/v {tuple(k.shape)} / {tuple(v.shape)} do not match the cache {tuple(k_cache.shape)}")
    if k.stride(-1) != 1 or v.stride() != k.stride():  # one set of source strides for both
        k, v = k.contiguous(), v.contiguous()
    slots = None
    if slot_indices is not None:
        slots = slot_indices.to(device=k.device, dtype=torch.int64)
        if slots.dim() != 1 or slots.shape[0] != B:
            raise ValueError(f"slot_indices must be [{B}]")
        slots = slots.contiguous()
    n_slots, Lmax = int(k_cache.shape[0]), int(k_cache.shape[1])
    rc = _lib.load().wdrz_kv_fill(
        _FILL_DTYPES[k.dtype], k.data_ptr(), v.data_ptr(), (_lib.ctypes.c_int64 * 3)(*k.stride()[:3]),
        k_cache.data_ptr(), v_cache.data_ptr(), (_lib.ctypes.c_int64 * 3)(*k_cache.stride()[:3]),
        slots.data_ptr() if slots is not None else None, B, T, H, D, n_slots, Lmax, int(start_pos),
        _stream_handle(),
    )
    if rc != _lib.WDRZ_OK:
        _raise(rc, "kv_fill")
    return True


class FlashKVCache:
    """Per-layer slot cache with the reference API (model.py:98-192), head-major storage.

    ``k_cache``/``v_cache`` are ``[batch_size, max_seq_length, n_heads, head_dim]`` views of
    ``[batch_size, n_heads, max_seq_length, head_dim]`` storage. Pass ``k_storage`` /
    ``v_storage`` (head-major tensors) to place the cache inside an existing arena.
    """

    def __init__(
        self,
        batch_size: int,
        max_seq_length: int,
        n_heads: int,
        head_dim: int,
        dtype=torch.float16,
        device=None,
        *,
        k_storage: Optional[Tensor] = None,
        v_storage: Optional[Tensor] = None,
        seq_lens: Optional[Tensor] = None,
    ):
        self.batch_size = batch_size
        self.max_seq_length = max_seq_length
        self.n_heads = n_heads
        self.head_dim = head_dim
        shape_hm = (batch_size, n_heads, max_seq_length, head_dim)
        if k_storage is None:
            k_storage = torch.zeros(shape_hm, dtype=dtype, device=device)
            v_storage = torch.zeros(shape_hm, dtype=dtype, device=device)
        if tuple(k_storage.shape) != shape_hm or tuple(v_storage.shape) != shape_hm:
            raise ValueError(f"storage must have head-major shape {shape_hm}")
        self.k_storage = k_storage
        self.v_storage = v_storage
        self.k_cache = k_storage.permute(0, 2, 1, 3)
        self.v_cache = v_storage.permute(0, 2, 1, 3)
        if seq_lens is None:
            seq_lens = torch.zeros(batch_size, dtype=torch.int32, device=k_storage.device)
        self.seq_lens = seq_lens
        self.done = False
        self.cross_attn_len = 0

    @property
    def dtype(self) -> torch.dtype:
        return self.k_storage.dtype

    @property
    def device(self) -> torch.device:
        return self.k_storage.device

    def prefill(self, k: Tensor, v: Tensor, start_pos: int = 0, slot_indices: Optional[Tensor] = None):
        """Write ``k, v`` ``[B, seq, heads, head_dim]`` at ``start_pos`` and set ``seq_lens``
        to the end position (model.py:150-168)."""
        seq_len = k.shape[1]
        end_pos = start_pos + seq_len
        written = _hip_fill(self.k_cache, self.v_cache, k, v, slot_indices, start_pos)
        if slot_indices is not None:
            if not written:
                self.k_cache[slot_indices, start_pos:end_pos] = k
                self.v_cache[slot_indices, start_pos:end_pos] = v
            self.seq_lens[slot_indices] = end_pos
        else:
            B = k.shape[0]
            if not written:
                self.k_cache[:B, start_pos:end_pos] = k
                self.v_cache[:B, start_pos:end_pos] = v
            self.seq_lens[:B] = end_pos

    def set_cross_attention(self, k: Tensor, v: Tensor, slot_indices: Optional[Tensor] = None):
        """Write the encoder-side ``k, v`` ``[B, seq, heads, head_dim]`` (model.py:170-183)."""
        seq_len = k.shape[1]
        if not _hip_fill(self.k_cache, self.v_cache, k, v, slot_indices, 0):
            if slot_indices is not None:
                self.k_cache[slot_indices, :seq_len] = k
                self.v_cache[slot_indices, :seq_len] = v
            else:
                B = k.shape[0]
                self.k_cache[:B, :seq_len] = k
                self.v_cache[:B, :seq_len] = v
        self.cross_attn_len = seq_len
        self.done = True

    def reset(self, slot_indices: Optional[Tensor] = None):
        """Zero the lengths of ``slot_indices`` (all slots if None); K/V are not cleared
        (model.py:185-192)."""
        if slot_indices is not None:
            self.seq_lens[slot_indices] = 0
        else:
            self.seq_lens.zero_()
        self.done = False
        self.cross_attn_len = 0


@dataclass(frozen=True)
class SlotPlan:
    n_slots: int
    bytes_per_slot: int
    total_bytes: int


def cache_bytes_per_slot(n_layers: int, n_heads: int, head_dim: int, self_len: int, cross_len: int,
                         dtype: torch.dtype) -> int:
    e = torch.empty((), dtype=dtype).element_size()
    return n_layers * 2 * n_heads * head_dim * e * (self_len + cross_len)


def plan_slots(hbm_budget_bytes: int, n_layers: int = 32, n_heads: int = 20, head_dim: int = 64,
               self_len: int = 448, cross_len: int = 1500, dtype: torch.dtype = torch.bfloat16) -> SlotPlan:
    """How many decode slots a KV arena of ``hbm_budget_bytes`` holds at these sizes."""
    per = cache_bytes_per_slot(n_layers, n_heads, head_dim, self_len, cross_len, dtype)
    # every per-layer slice is rounded up to the arena alignment
    n = max(0, hbm_budget_bytes // per)
    while n > 0 and KVSlotPool.arena_bytes(n, n_layers, n_heads, head_dim, self_len, cross_len, dtype) > hbm_budget_bytes:
        n -= 1
    return SlotPlan(n_slots=int(n), bytes_per_slot=per,
                    total_bytes=KVSlotPool.arena_bytes(n, n_layers, n_heads, head_dim, self_len, cross_len, dtype))


class KVSlotPool:
    """All layers' self and cross caches in one arena (replaces ``create_flash_kv``,
    model.py:773-808, and ``reset_flash_kv``, model.py:810-822).

    ``self_kv[l]`` / ``cross_kv[l]`` are ``FlashKVCache`` objects whose storage are slices of
    the arena. Self caches of all layers share nothing but the arena; each layer keeps its
    own ``seq_lens`` as in the reference, stored as row ``l`` of one ``[n_layers, n_slots]``
    int32 tensor (``self_seq_lens``) so that a decode step can gather and bump every layer's
    lengths with one operation each.
    """

    def __init__(self, n_layers: int, n_slots: int, n_heads: int = 20, head_dim: int = 64,
                 self_len: int = 448, cross_len: int = 1500, dtype: torch.dtype = torch.bfloat16,
                 device=None):
        self.n_layers, self.n_slots = n_layers, n_slots
        self.n_heads, self.head_dim = n_heads, head_dim
        self.self_len, self.cross_len = self_len, cross_len
        self.dtype = dtype
        nbytes = self.arena_bytes(n_slots, n_layers, n_heads, head_dim, self_len, cross_len, dtype)
        self.arena = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        e = torch.empty((), dtype=dtype).element_size()
        off = 0

        def take(seq_len: int) -> Tensor:
            nonlocal off
            n = n_slots * n_heads * seq_len * head_dim * e
            t = self.arena[off : off + n].view(dtype).view(n_slots, n_heads, seq_len, head_dim)
            off += (n + _ALIGN - 1) // _ALIGN * _ALIGN
            return t

        self.self_kv: list[FlashKVCache] = []
        self.cross_kv: list[FlashKVCache] = []
        self.self_seq_lens = torch.zeros((n_layers, n_slots), dtype=torch.int32, device=self.arena.device)
        for l in range(n_layers):
            ks, vs = take(self_len), take(self_len)
            self.self_kv.append(FlashKVCache(n_slots, self_len, n_heads, head_dim, k_storage=ks, v_storage=vs,
                                             seq_lens=self.self_seq_lens[l]))
            kx, vx = take(cross_len), take(cross_len)
            self.cross_kv.append(FlashKVCache(n_slots, cross_len, n_heads, head_dim, k_storage=kx, v_storage=vx))

    @staticmethod
    def arena_bytes(n_slots: int, n_layers: int, n_heads: int, head_dim: int, self_len: int, cross_len: int,
                    dtype: torch.dtype) -> int:
        e = torch.empty((), dtype=dtype).element_size()

        def rounded(seq_len: int) -> int:
            n = n_slots * n_heads * seq_len * head_dim * e
            return (n + _ALIGN - 1) // _ALIGN * _ALIGN

        return n_layers * 2 * (rounded(self_len) + rounded(cross_len))

    def reset(self, slot_indices: Optional[Tensor] = None) -> None:
        for s_kv, c_kv in zip(self.self_kv, self.cross_kv, strict=True):
            s_kv.reset(slot_indices)
            c_kv.reset(slot_indices)
