"""Fused small operations of the decode step, backed by the gfx950 kernels in libwdrz_attn.so.

* :func:`add_layernorm_` — ``x += delta; return ln(x)``: the residual add closing a sub-layer
  and the LayerNorm opening the next (reference ``src/whisperdrz/model.py:420-433``, the final
  ``ln`` at ``model.py:609-613``), one launch instead of two.
* :func:`masked_argmax` — ``decode_batch``'s greedy sampling tail (``decoding.py:1729-1761``):
  additive -65504 mask, repetition penalty, argmax, one launch instead of six.
* :func:`linear_gelu` — the MLP's ``Linear(n_state, 4 n_state)`` + ``GELU`` (``model.py:388-391``,
  applied at ``model.py:434``): GEMM, bias, rounding and exact GELU in one launch.

There is no fallback: CPU tensors, fp32 LayerNorm inputs and a missing library raise.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from . import _lib
from .attention import _check_cuda, _dtype_code, _raise, _stream_handle

__all__ = ["add_layernorm_", "layer_norm", "linear_gelu", "masked_argmax"]

_LN16 = {torch.bfloat16: _lib.WDRZ_BF16, torch.float16: _lib.WDRZ_F16}


def _rows(t: torch.Tensor, name: str) -> torch.Tensor:
    r = t.reshape(-1, t.shape[-1])
    if r.stride(-1) != 1 or r.data_ptr() != t.data_ptr():
        raise ValueError(f"{name} must have contiguous rows")
    return r


def add_layernorm_(x: torch.Tensor, delta: Optional[torch.Tensor], ln: nn.LayerNorm) -> torch.Tensor:
    """In place ``x += delta`` (when ``delta`` is given), then returns ``ln(x)`` (fp32 statistics)."""
    _check_cuda("x", x, x.device)
    if x.dtype not in _LN16:
        raise TypeError(f"x: dtype {x.dtype} is not supported (bfloat16, float16)")
    xr = _rows(x, "x")
    dr = None
    if delta is not None:
        _check_cuda("delta", delta, x.device)
        if delta.dtype != x.dtype or delta.shape != x.shape:
            raise ValueError("delta must match x in shape and dtype")
        dr = delta.reshape(xr.shape) if delta.is_contiguous() else delta.contiguous().reshape(xr.shape)
    w = ln.weight.detach()
    b = ln.bias.detach()
    if w.dtype != x.dtype:
        raise TypeError("the LayerNorm parameters must have the activations' dtype")
    y = torch.empty_like(xr)
    rc = _lib.load().wdrz_add_layernorm(
        _LN16[x.dtype], xr.data_ptr(), xr.stride(0), dr.data_ptr() if dr is not None else None,
        dr.stride(0) if dr is not None else 0, w.data_ptr(), b.data_ptr(), y.data_ptr(), y.stride(0),
        xr.shape[0], xr.shape[1], float(ln.eps), _stream_handle(),
    )
    if rc != _lib.WDRZ_OK:
        _raise(rc, "add_layernorm_")
    return y.view(x.shape)


def layer_norm(x: torch.Tensor, ln: nn.LayerNorm) -> torch.Tensor:
    return add_layernorm_(x, None, ln)


def masked_argmax(logits: torch.Tensor, blocked: Optional[torch.Tensor] = None,
                  penalty: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Greedy token per row of ``logits [rows, V]`` under the bool ``blocked`` mask (additive
    -65504) and the bool ``penalty`` mask (repetition penalty 1.2), as decode_batch computes it."""
    _check_cuda("logits", logits, logits.device)
    if logits.dim() == 3:
        logits = logits[:, -1, :]
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    rows, V = (int(v) for v in logits.shape)
    out = torch.empty(rows, dtype=torch.long, device=logits.device)
    masks = []
    for name, m in (("blocked", blocked), ("penalty", penalty)):
        if m is None:
            masks.append((None, 0))
            continue
        _check_cuda(name, m, logits.device)
        if m.dtype != torch.bool or m.shape[-1] < V or m.dim() != 2 or m.stride(-1) != 1:
            raise ValueError(f"{name} must be a bool [rows, >= V] tensor with contiguous rows")
        masks.append((m, m.stride(0)))
    rc = _lib.load().wdrz_masked_argmax(
        _dtype_code(logits, "logits"), logits.data_ptr(), logits.stride(0),
        masks[0][0].data_ptr() if masks[0][0] is not None else None, masks[0][1],
        masks[1][0].data_ptr() if masks[1][0] is not None else None, masks[1][1],
        out.data_ptr(), rows, V, _stream_handle(),
    )
    if rc != _lib.WDRZ_OK:
        _raise(rc, "masked_argmax")
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], gelu: bool = False) -> torch.Tensor:
    """``x @ weight.T + bias`` (``gelu``: then the exact GELU) for 16-bit ``x [..., K]``, rounded
    like torch's 16-bit modules: the Linear's output to the storage type, then the GELU's."""
    _check_cuda("x", x, x.device)
    if x.dtype not in _LN16:
        raise TypeError(f"x: dtype {x.dtype} is not supported (bfloat16, float16)")
    xr = _rows(x, "x")
    w = weight.detach()
    b = bias.detach() if bias is not None else None
    if w.dtype != x.dtype or (b is not None and b.dtype != x.dtype):
        raise TypeError("the Linear's parameters must have the activations' dtype")
    if w.stride(-1) != 1 or w.shape[1] != xr.shape[1]:
        raise ValueError("weight must be [N, K] with contiguous rows and K = x.shape[-1]")
    if b is not None and not b.is_contiguous():
        b = b.contiguous()
    N = int(w.shape[0])
    y = torch.empty(xr.shape[0], N, dtype=x.dtype, device=x.device)
    rc = _lib.load().wdrz_linear(
        _LN16[x.dtype], xr.data_ptr(), xr.stride(0), w.data_ptr(), w.stride(0),
        b.data_ptr() if b is not None else None, y.data_ptr(), y.stride(0),
        xr.shape[0], N, xr.shape[1], 1 if gelu else 0, _stream_handle(),
    )
    if rc != _lib.WDRZ_OK:
        _raise(rc, "linear")
    return y.view(*x.shape[:-1], N)


def linear_gelu(x: torch.Tensor, lin: nn.Linear, gelu: bool = True) -> torch.Tensor:
    """``GELU(lin(x))`` (``gelu=False``: ``lin(x)``) for 16-bit ``x [..., K]``, rounded like the
    reference's two modules: the Linear's output to the storage type, then the GELU's."""
    return linear(x, lin.weight, lin.bias, gelu)


def linear_partials(x: torch.Tensor, lin: nn.Linear, n_split: int = 4) -> torch.Tensor:
    """fp32 split-K partial products of ``lin`` (no bias) for 16-bit ``x [..., K]``: a tensor
    ``[n_split, rows, N]`` whose sum over the first dimension is ``x @ lin.weight.T``; its
    consumer (``add_layernorm_partials_``) adds the bias and rounds like the Linear's output."""
    _check_cuda("x", x, x.device)
    if x.dtype not in _LN16:
        raise TypeError(f"x: dtype {x.dtype} is not supported (bfloat16, float16)")
    xr = _rows(x, "x")
    w = lin.weight.detach()
    if w.dtype != x.dtype:
        raise TypeError("the Linear's parameters must have the activations' dtype")
    if w.stride(-1) != 1 or w.shape[1] != xr.shape[1]:
        raise ValueError("weight must be [N, K] with contiguous rows and K = x.shape[-1]")
    N = int(w.shape[0])
    part = torch.empty(n_split, xr.shape[0], N, dtype=torch.float32, device=x.device)
    rc = _lib.load().wdrz_linear_partials(
        _LN16[x.dtype], xr.data_ptr(), xr.stride(0), w.data_ptr(), w.stride(0), part.data_ptr(),
        xr.shape[0], N, xr.shape[1], n_split, _stream_handle(),
    )
    if rc != _lib.WDRZ_OK:
        _raise(rc, "linear_partials")
    return part


def add_layernorm_partials_(x: torch.Tensor, partials: torch.Tensor, lin: nn.Linear,
                            ln: nn.LayerNorm) -> torch.Tensor:
    """In place ``x += lin(h)`` where ``partials = linear_partials(h, lin)`` (the sum of the
    partials plus ``lin.bias``, rounded to ``x``'s type like the Linear's output), then returns
    ``ln(x)`` as ``add_layernorm_`` does."""
    _check_cuda("x", x, x.device)
    if x.dtype not in _LN16:
        raise TypeError(f"x: dtype {x.dtype} is not supported (bfloat16, float16)")
    xr = _rows(x, "x")
    n_split = int(partials.shape[0])
    if partials.dtype != torch.float32 or tuple(partials.shape[1:]) != tuple(xr.shape) or not partials.is_contiguous():
        raise ValueError("partials must be contiguous fp32 [n_split, rows, n] matching x")
    if lin.bias is None:
        raise ValueError("the Linear must have a bias")
    db = lin.bias.detach()
    w = ln.weight.detach()
    b = ln.bias.detach()
    if w.dtype != x.dtype or db.dtype != x.dtype:
        raise TypeError("the LayerNorm and Linear parameters must have the activations' dtype")
    y = torch.empty_like(xr)
    rc = _lib.load().wdrz_add_layernorm_partials(
        _LN16[x.dtype], xr.data_ptr(), xr.stride(0), partials.data_ptr(), n_split, db.data_ptr(),
        w.data_ptr(), b.data_ptr(), y.data_ptr(), y.stride(0), xr.shape[0], xr.shape[1], float(ln.eps),
        _stream_handle(),
    )
    if rc != _lib.WDRZ_OK:
        _raise(rc, "add_layernorm_partials_")
    return y.view(x.shape)
