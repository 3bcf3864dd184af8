"""Decoder plumbing around the attention hot path: the callers of the two seams.

This mirrors, with random weights and no tokenizer, the pieces of the reference that call the
cached attention, so the HIP kernels can be exercised exactly as WhisperDRZ drives them:

* ``MultiHeadAttention.forward_flash`` — projections, ``cache_seqlens = seq_lens[slots]``,
  int32 ``cache_batch_idx``, scale ``head_dim**-0.5``, then the seam
  (reference ``src/whisperdrz/model.py:301-362``); ``forward`` is the uncached path through
  ``qkv_attention`` (model.py:265-298).
* ``ResidualAttentionBlock`` — pre-LN self-attention, cross-attention, GELU MLP
  (model.py:365-434).
* ``TextDecoderStack.forward_flash`` / ``prefill_flash`` — embeddings, the blocks, the
  ``seq_lens`` bump after all layers, final LN and tied-embedding logits (model.py:570-617,
  824-869).
* ``TextDecoderStack._fused_blocks`` — the same blocks with each residual add fused into the
  next LayerNorm (``decode_ops.add_layernorm_``), the step's metadata (int32 slot map, every
  layer's gathered lengths) computed once per step, the self-attention query / key / value
  projections as one GEMM (``decode_ops.linear``), fc1 with its GELU as one kernel
  (``linear_gelu``), and the attention output projections and fc2 as split-K partials summed by
  the residual add (``linear_partials`` + ``add_layernorm_partials_``); the default for 16-bit
  GPU activations.
* ``BucketedDecodeGraphs`` — one captured decode step per batch bucket, replayed with static
  token / position / slot buffers (reference ``transcriber.py:18-173``); on ROCm
  ``torch.cuda.CUDAGraph`` is a hipGraph.

The attention functions are injectable (``attn_kvcache`` / ``attn_dense``) so a test can run
the same stack against the reference's torch arithmetic; by default they are the HIP kernels.
"""
from __future__ import annotations

from collections import defaultdict
from typing import Callable, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from .attention import flash_attn_with_kvcache, scaled_dot_product_attention
from .decode_ops import add_layernorm_, add_layernorm_partials_, layer_norm, linear, linear_gelu, linear_partials
from .kv_cache import FlashKVCache, KVSlotPool

# Batch buckets of the captured decode step (reference transcriber.py:18).
GRAPH_BUCKETS = [1, 2, 4, 8, 16, 32, 42, 52, 54]


def bucket_for(batch: int, buckets: list[int]) -> int:
    """Smallest bucket >= batch, or batch itself when none fits (reference transcriber.py:21-28)."""
    for b in buckets:
        if batch <= b:
            return b
    return batch


def _out_add_layernorm(x: Tensor, o: Tensor, out: nn.Linear, ln: nn.LayerNorm) -> Tensor:
    """``x += out(o)`` then ``ln(x)`` (the output projection at model.py:362, the residual adds at
    420-432 and the next sub-layer's LayerNorm): the
    attention's output projection as 2 split-K fp32 partials summed by the residual add (K a
    multiple of 256, n_state <= 1536), else torch's Linear and the fused add + LayerNorm."""
    if out.in_features % 256 == 0 and out.out_features <= 1536 and out.bias is not None:
        return add_layernorm_partials_(x, linear_partials(o, out, 2), out, ln)
    return add_layernorm_(x, out(o), ln)


def lengths_matrix(self_kv: list[FlashKVCache]) -> Optional[Tensor]:
    """The ``[n_layers, n_slots]`` tensor whose row ``l`` is ``self_kv[l].seq_lens`` (as
    ``KVSlotPool`` lays them out), or None when the layers' lengths are separate tensors."""
    base = self_kv[0].seq_lens._base if self_kv else None
    if base is None or base.dim() != 2 or base.shape[0] != len(self_kv) or not base.is_contiguous():
        return None
    for l, s in enumerate(self_kv):
        if s.seq_lens._base is not base or s.seq_lens.data_ptr() != base[l].data_ptr() or s.seq_lens.shape != base[l].shape:
            return None
    return base


class MultiHeadAttention(nn.Module):
    def __init__(self, n_state: int, n_head: int, causal: bool = False,
                 attn_kvcache: Callable = flash_attn_with_kvcache, attn_dense: Callable = scaled_dot_product_attention):
        super().__init__()
        self.n_state, self.n_head, self.causal = n_state, n_head, causal
        self.query = nn.Linear(n_state, n_state)
        self.key = nn.Linear(n_state, n_state, bias=False)
        self.value = nn.Linear(n_state, n_state)
        self.out = nn.Linear(n_state, n_state)
        self.attn_kvcache = attn_kvcache
        self.attn_dense = attn_dense

    def forward(self, x: Tensor, xa: Optional[Tensor] = None) -> Tensor:
        """Uncached attention (encoder, DTW decoder): SDPA over [B, h, T, d] views."""
        src = x if xa is None else xa
        q, k, v = self.query(x), self.key(src), self.value(src)
        B, T, _ = q.shape
        d = self.n_state // self.n_head
        heads = lambda t: t.view(t.shape[0], t.shape[1], self.n_head, d).permute(0, 2, 1, 3)
        scale = d ** -0.25
        o = self.attn_dense(heads(q), heads(k), heads(v), is_causal=self.causal and T > 1, scale=scale * scale)
        return self.out(o.permute(0, 2, 1, 3).reshape(B, T, self.n_state))

    def qkv_weight(self) -> tuple[Tensor, Tensor]:
        """``[query; key; value]`` weights ``[3*n_state, n_state]`` and bias (the key's part zero)
        as one projection, rebuilt whenever a parameter is replaced or modified in place."""
        ps = (self.query.weight, self.key.weight, self.value.weight, self.query.bias, self.value.bias)
        key = tuple((p.data_ptr(), p._version, p.dtype) for p in ps)
        cached = getattr(self, "_qkv_cache", None)
        if cached is None or cached[0] != key:
            with torch.no_grad():
                w = torch.cat([self.query.weight, self.key.weight, self.value.weight])
                b = torch.cat([self.query.bias, torch.zeros_like(self.query.bias), self.value.bias])
            cached = (key, w, b)
            self._qkv_cache = cached
        return cached[1], cached[2]

    def kv_weight(self) -> tuple[Tensor, Tensor]:
        """``[key; value]`` weights ``[2*n_state, n_state]`` and bias (the key's part zero): the
        cross-attention fill's two projections of the encoder output as one GEMM."""
        ps = (self.key.weight, self.value.weight, self.value.bias)
        key = tuple((p.data_ptr(), p._version, p.dtype) for p in ps)
        cached = getattr(self, "_kv_cache", None)
        if cached is None or cached[0] != key:
            with torch.no_grad():
                w = torch.cat([self.key.weight, self.value.weight])
                b = torch.cat([torch.zeros_like(self.value.bias), self.value.bias])
            cached = (key, w, b)
            self._kv_cache = cached
        return cached[1], cached[2]

    def forward_flash_step(self, x: Tensor, kv_cache: FlashKVCache, is_cross_attn: bool,
                           cache_seqlens: Optional[Tensor], batch_idx: Optional[Tensor],
                           project_out: bool = True) -> Tensor:
        """``forward_flash`` with the step's metadata computed once by the caller (the gathered
        ``cache_seqlens`` and the int32 slot map) and, for self-attention, the query / key /
        value projections as one GEMM (``decode_ops.linear`` when K % 128 == 0, as is the
        cross-attention's query projection). Same arithmetic per output element.
        ``project_out=False`` returns the attention output before ``out`` (the caller applies it,
        fused with the residual add)."""
        B, seq_len, _ = x.shape
        d = self.n_state // self.n_head
        if is_cross_attn:
            # the query projection on the same 64-row kernel as the others (K % 128 == 0)
            q = linear(x, self.query.weight, self.query.bias) if self.n_state % 128 == 0 else self.query(x)
            q = q.view(B, seq_len, self.n_head, d)
            o = self.attn_kvcache(q, kv_cache.k_cache, kv_cache.v_cache, cache_batch_idx=batch_idx,
                                  softmax_scale=d ** -0.5, causal=False)
        else:
            w, b = self.qkv_weight()
            qkv = linear(x, w, b) if self.n_state % 128 == 0 else F.linear(x, w, b)
            qkv = qkv.view(B, seq_len, 3, self.n_head, d)
            o = self.attn_kvcache(qkv[:, :, 0], kv_cache.k_cache, kv_cache.v_cache, k=qkv[:, :, 1], v=qkv[:, :, 2],
                                  cache_seqlens=cache_seqlens, cache_batch_idx=batch_idx, softmax_scale=d ** -0.5,
                                  causal=self.causal)
        o = o.reshape(B, seq_len, self.n_state)
        return self.out(o) if project_out else o

    def forward_flash(self, x: Tensor, kv_cache: FlashKVCache, is_cross_attn: bool = False,
                      slot_indices: Optional[Tensor] = None) -> Tensor:
        B, seq_len, _ = x.shape
        d = self.n_state // self.n_head
        q = self.query(x).view(B, seq_len, self.n_head, d)
        seqlens = kv_cache.seq_lens if slot_indices is None else kv_cache.seq_lens[slot_indices]
        batch_idx = None if slot_indices is None else slot_indices.to(torch.int32)
        if is_cross_attn:
            o = self.attn_kvcache(q, kv_cache.k_cache, kv_cache.v_cache, cache_batch_idx=batch_idx,
                                  softmax_scale=d ** -0.5, causal=False)
        else:
            k_new = self.key(x).view(B, seq_len, self.n_head, d)
            v_new = self.value(x).view(B, seq_len, self.n_head, d)
            o = self.attn_kvcache(q, kv_cache.k_cache, kv_cache.v_cache, k=k_new, v=v_new, cache_seqlens=seqlens,
                                  cache_batch_idx=batch_idx, softmax_scale=d ** -0.5, causal=self.causal)
        return self.out(o.reshape(B, seq_len, self.n_state))


class ResidualAttentionBlock(nn.Module):
    def __init__(self, n_state: int, n_head: int, **attn_kw):
        super().__init__()
        self.attn = MultiHeadAttention(n_state, n_head, causal=True, **attn_kw)
        self.attn_ln = nn.LayerNorm(n_state)
        self.cross_attn = MultiHeadAttention(n_state, n_head, causal=False, **attn_kw)
        self.cross_attn_ln = nn.LayerNorm(n_state)
        self.mlp = nn.Sequential(nn.Linear(n_state, 4 * n_state), nn.GELU(), nn.Linear(4 * n_state, n_state))
        self.mlp_ln = nn.LayerNorm(n_state)

    def forward(self, x: Tensor, xa: Tensor) -> Tensor:
        x = x + self.attn(self.attn_ln(x))
        x = x + self.cross_attn(self.cross_attn_ln(x), xa)
        return x + self.mlp(self.mlp_ln(x))

    def forward_flash(self, x: Tensor, self_kv: FlashKVCache, cross_kv: FlashKVCache,
                      slot_indices: Optional[Tensor] = None) -> Tensor:
        x = x + self.attn.forward_flash(self.attn_ln(x), self_kv, is_cross_attn=False, slot_indices=slot_indices)
        x = x + self.cross_attn.forward_flash(self.cross_attn_ln(x), cross_kv, is_cross_attn=True,
                                              slot_indices=slot_indices)
        return x + self.mlp(self.mlp_ln(x))


class TextDecoderStack(nn.Module):
    """Token embedding + positional embedding, ``n_layer`` blocks, LN, tied logits."""

    def __init__(self, n_vocab: int, n_ctx: int, n_state: int, n_head: int, n_layer: int, **attn_kw):
        super().__init__()
        self.n_ctx, self.n_state, self.n_head, self.n_layer = n_ctx, n_state, n_head, n_layer
        self.token_embedding = nn.Embedding(n_vocab, n_state)
        self.positional_embedding = nn.Parameter(torch.randn(n_ctx, n_state) * 0.02)
        self.blocks = nn.ModuleList([ResidualAttentionBlock(n_state, n_head, **attn_kw) for _ in range(n_layer)])
        self.ln = nn.LayerNorm(n_state)
        # Cached steps on 16-bit GPU activations fuse every residual add with the LayerNorm that
        # follows it (one kernel instead of two); False keeps torch's separate ops.
        self.fused_small_ops = True

    def forward(self, tokens: Tensor, xa: Tensor) -> Tensor:
        """Uncached forward over all tokens (the DTW-alignment path, model.py:547-568)."""
        x = self.token_embedding(tokens) + self.positional_embedding[: tokens.shape[1]]
        for block in self.blocks:
            x = block(x, xa)
        return self.ln(x) @ self.token_embedding.weight.to(x.dtype).T

    def forward_flash(self, tokens: Tensor, self_kv: list[FlashKVCache], cross_kv: list[FlashKVCache],
                      positions: Tensor, slot_indices: Optional[Tensor] = None) -> Tensor:
        B, seq_len = tokens.shape
        if positions.dim() == 1:
            positions = positions.unsqueeze(1).expand(B, seq_len)
        x = self.token_embedding(tokens) + self.positional_embedding[positions]
        if self.fused_small_ops and x.is_cuda and x.dtype in (torch.bfloat16, torch.float16):
            h = self._fused_blocks(x.contiguous(), self_kv, cross_kv, slot_indices)
        else:
            for block, s_kv, c_kv in zip(self.blocks, self_kv, cross_kv, strict=True):
                x = block.forward_flash(x, s_kv, c_kv, slot_indices=slot_indices)
            h = self.ln(x)
        # the attention never bumps lengths; the caller does, after all layers
        lens = lengths_matrix(self_kv)
        if lens is not None:  # every layer's row at once, same indexing as per layer
            if slot_indices is not None:
                lens[:, slot_indices] += seq_len
            else:
                lens[:, :B] += seq_len
        else:
            for s_kv in self_kv:
                if slot_indices is not None:
                    s_kv.seq_lens[slot_indices] += seq_len
                else:
                    s_kv.seq_lens[:B] += seq_len
        return h @ self.token_embedding.weight.to(h.dtype).T

    def _fused_blocks(self, x: Tensor, self_kv: list[FlashKVCache], cross_kv: list[FlashKVCache],
                      slot_indices: Optional[Tensor]) -> Tensor:
        """The blocks of ``forward_flash`` with each residual add fused into the next LayerNorm
        (model.py:420-433): x is the residual stream, updated in place; returns ln(x)."""
        blocks = list(self.blocks)
        # the step's metadata once, not per layer: the int32 slot map and every layer's gathered
        # self lengths (one gather from the [n_layers, n_slots] lengths when the layers' lengths
        # are its rows)
        B = x.shape[0]
        batch_idx = None if slot_indices is None else slot_indices.to(torch.int32)
        lens = lengths_matrix(self_kv)
        if lens is not None:
            seqlens = (lens[:, slot_indices] if slot_indices is not None else lens[:, :B]).contiguous()
            layer_lens = [seqlens[i] for i in range(len(blocks))]
        else:
            layer_lens = [s.seq_lens if slot_indices is None else s.seq_lens[slot_indices] for s in self_kv]
        h = layer_norm(x, blocks[0].attn_ln)
        for i, (block, s_kv, c_kv) in enumerate(zip(blocks, self_kv, cross_kv, strict=True)):
            o = block.attn.forward_flash_step(h, s_kv, False, layer_lens[i], batch_idx, project_out=False)
            h = _out_add_layernorm(x, o, block.attn.out, block.cross_attn_ln)
            o = block.cross_attn.forward_flash_step(h, c_kv, True, None, batch_idx, project_out=False)
            h = _out_add_layernorm(x, o, block.cross_attn.out, block.mlp_ln)
            fc1, fc2 = block.mlp[0], block.mlp[2]
            ln_next = blocks[i + 1].attn_ln if i + 1 < len(blocks) else self.ln
            # fused fc1 + GELU, then fc2 as 4 split-K fp32 partials that the residual add sums
            # (with fc2's bias and rounding) before the next LayerNorm: every Whisper width
            # (K % 128 == 0, 4 K % 512 == 0, n <= 1536); other widths keep torch's MLP
            if fc1.in_features % 128 == 0 and fc2.in_features % 512 == 0 and fc2.out_features <= 1536 \
                    and fc2.bias is not None:
                h = add_layernorm_partials_(x, linear_partials(linear_gelu(h, fc1), fc2, 4), fc2, ln_next)
            else:
                h = add_layernorm_(x, block.mlp(h), ln_next)
        return h

    def prefill_flash(self, tokens: Tensor, xa: Tensor, self_kv: list[FlashKVCache], cross_kv: list[FlashKVCache],
                      slot_indices: Optional[Tensor] = None) -> Tensor:
        """Project the encoder output into every layer's cross cache, zero the self lengths and
        run the prompt as one multi-token causal step (model.py:824-869)."""
        B, seq_len = tokens.shape
        d = self.n_state // self.n_head
        fused = self.fused_small_ops and xa.is_cuda and xa.dtype in (torch.bfloat16, torch.float16)
        for block, c_kv in zip(self.blocks, cross_kv, strict=True):
            if fused:  # key and value projections as one [B*T, n_state] x [n_state, 2*n_state] GEMM
                w, b = block.cross_attn.kv_weight()
                kv = F.linear(xa, w, b).view(B, -1, 2, self.n_head, d)
                k, v = kv[:, :, 0], kv[:, :, 1]
            else:
                k = block.cross_attn.key(xa).view(B, -1, self.n_head, d)
                v = block.cross_attn.value(xa).view(B, -1, self.n_head, d)
            c_kv.set_cross_attention(k, v, slot_indices)
        for s_kv in self_kv:
            if slot_indices is not None:
                s_kv.seq_lens[slot_indices] = 0
            else:
                s_kv.seq_lens[:B] = 0
        positions = torch.arange(seq_len, device=tokens.device).unsqueeze(0).expand(B, -1)
        return self.forward_flash(tokens, self_kv, cross_kv, positions, slot_indices)


class BucketedDecodeGraphs:
    """Captured single-token decode steps per batch bucket (reference transcriber.py:31-173).

    Padded rows of a bucket keep the slot ids they were captured or last called with, as in the
    reference, so callers that pad must make those slots harmless (the reference's own
    behaviour: padded rows append into, and bump the lengths of, those slots).
    """

    def __init__(self, decoder: TextDecoderStack, pool: KVSlotPool, n_vocab: int, buckets: Optional[list[int]] = None):
        self.decoder, self.pool, self.n_vocab = decoder, pool, n_vocab
        self.buckets = list(buckets if buckets is not None else GRAPH_BUCKETS)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.static: dict[int, dict[str, Tensor]] = {}
        self.hits: defaultdict[int, int] = defaultdict(int)
        self.misses = 0

    def _step(self, bucket: int) -> Tensor:
        st = self.static[bucket]
        return self.decoder.forward_flash(st["tokens"], self.pool.self_kv, self.pool.cross_kv, st["positions"],
                                          slot_indices=st["slots"])

    def capture(self, bucket: int) -> None:
        dev = self.pool.arena.device
        self.static[bucket] = {
            "tokens": torch.zeros(bucket, 1, dtype=torch.long, device=dev),
            "positions": torch.zeros(bucket, dtype=torch.long, device=dev),
            "slots": torch.arange(bucket, dtype=torch.long, device=dev),
        }
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                self._step(bucket)
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.static[bucket]["logits"] = self._step(bucket)
        self.graphs[bucket] = g

    def forward(self, tokens: Tensor, positions: Tensor, slot_indices: Tensor) -> Tensor:
        B = tokens.shape[0]
        bucket = bucket_for(B, self.buckets)
        if bucket not in self.graphs:
            self.misses += 1
            return self.decoder.forward_flash(tokens, self.pool.self_kv, self.pool.cross_kv, positions,
                                              slot_indices=slot_indices)
        self.hits[bucket] += 1
        st = self.static[bucket]
        st["tokens"][:B].copy_(tokens)
        st["positions"][:B].copy_(positions)
        st["slots"][:B].copy_(slot_indices)
        self.graphs[bucket].replay()
        return st["logits"][:B]
