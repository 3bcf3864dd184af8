"""GPU parity of the fused decode-step operations (whisperdrz_amd.decode_ops) against the
reference's own torch ops on the same GPU tensors.

* add_layernorm_: the new residual x + delta bit-identical to torch's add; the LayerNorm within
  one unit in the last place of the 16-bit result of torch's LayerNorm (both compute in fp32;
  the reduction order differs), with at least 99% of the elements bit-identical.
* add_layernorm_partials_: the delta given as fp32 split-K partials of a Linear plus its bias; the
  reference is torch's sequential fp32 sum of the partials plus the bias, rounded to the 16-bit
  type (the Linear's output), then the same add and LayerNorm: the residual bit-identical, the
  LayerNorm to the bar above.
* masked_argmax: token ids identical to the reference's sequence (zero, masked_fill -65504, add,
  repetition-penalty where, argmax; decoding.py:1729-1761, 854-855), ties and NaN logits included
  (a NaN is the maximum, as in torch.argmax).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ulp16(t: torch.Tensor) -> torch.Tensor:
    bits = 7 if t.dtype == torch.bfloat16 else 10
    a = t.float().abs().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - bits)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,n", [(64, 1280), (3, 256), (130, 4096), (1, 8)])
def test_add_layernorm(cuda, dtype, rows, n):
    from whisperdrz_amd import add_layernorm_, layer_norm

    g = torch.Generator(device=cuda).manual_seed(rows + n)
    x = (3.0 * torch.randn(rows, n, generator=g, device=cuda) + 0.5).to(dtype)
    delta = torch.randn(rows, n, generator=g, device=cuda).to(dtype)
    ln = torch.nn.LayerNorm(n).to(cuda, dtype)
    with torch.no_grad():
        ln.weight.copy_(1.0 + 0.1 * torch.randn(n, generator=g, device=cuda))
        ln.bias.copy_(0.1 * torch.randn(n, generator=g, device=cuda))
    print(f"add_layernorm {dtype} rows={rows} n={n}", flush=True)
    x_ref = x + delta
    y_ref = ln(x_ref)
    x_in = x.clone()
    y = add_layernorm_(x_in, delta, ln)
    torch.cuda.synchronize()
    assert torch.equal(x_in, x_ref)  # the new residual, in place
    diff = (y.float() - y_ref.float()).abs()
    assert torch.all(diff <= _ulp16(y_ref) * 1.001), float(diff.max())
    assert (diff == 0).float().mean().item() >= 0.99
    # plain LayerNorm leaves x untouched
    x_keep = x.clone()
    y2 = layer_norm(x_keep, ln)
    assert torch.equal(x_keep, x)
    assert torch.all((y2.float() - ln(x).float()).abs() <= _ulp16(ln(x)) * 1.001)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,n,n_split", [(64, 1280, 4), (3, 256, 2), (130, 1536, 4), (1, 8, 4), (5, 1032, 2)])
def test_add_layernorm_partials(cuda, dtype, rows, n, n_split):
    from whisperdrz_amd import add_layernorm_partials_

    g = torch.Generator(device=cuda).manual_seed(rows * 5 + n + n_split)
    x = (3.0 * torch.randn(rows, n, generator=g, device=cuda) + 0.5).to(dtype)
    partials = torch.randn(n_split, rows, n, generator=g, device=cuda)
    fc = torch.nn.Linear(8, n).to(cuda, dtype)  # only its bias is used
    ln = torch.nn.LayerNorm(n).to(cuda, dtype)
    with torch.no_grad():
        fc.bias.copy_(0.5 * torch.randn(n, generator=g, device=cuda))
        ln.weight.copy_(1.0 + 0.1 * torch.randn(n, generator=g, device=cuda))
        ln.bias.copy_(0.1 * torch.randn(n, generator=g, device=cuda))
    print(f"add_layernorm_partials {dtype} rows={rows} n={n} n_split={n_split}", flush=True)
    acc = partials[0].clone()
    for z in range(1, n_split):
        acc = acc + partials[z]
    delta_ref = (acc + fc.bias.float()).to(dtype)
    x_ref = x + delta_ref
    y_ref = ln(x_ref)
    x_in = x.clone()
    y = add_layernorm_partials_(x_in, partials, fc, ln)
    torch.cuda.synchronize()
    assert torch.equal(x_in, x_ref)
    diff = (y.float() - y_ref.float()).abs()
    assert torch.all(diff <= _ulp16(y_ref) * 1.001), float(diff.max())
    assert (diff == 0).float().mean().item() >= 0.99


def test_add_layernorm_partials_errors(cuda):
    from whisperdrz_amd import add_layernorm_partials_

    x = torch.randn(4, 2048, device=cuda).to(torch.bfloat16)
    fc = torch.nn.Linear(8, 2048).to(cuda, torch.bfloat16)
    ln = torch.nn.LayerNorm(2048).to(cuda, torch.bfloat16)
    with pytest.raises(NotImplementedError, match="1536"):
        add_layernorm_partials_(x, torch.zeros(4, 4, 2048, device=cuda), fc, ln)
    with pytest.raises(ValueError):
        add_layernorm_partials_(x, torch.zeros(4, 3, 2048, device=cuda), fc, ln)


def _reference_sampling(logits, blocked, penalty):
    additive = torch.zeros_like(logits)
    if blocked is not None:
        additive.masked_fill_(blocked, -65504)
    masked = logits + additive
    if penalty is not None:
        penalized = torch.where(masked > 0, masked / 1.2, masked * 1.2)
        masked = torch.where(penalty, penalized, masked)
    return masked.argmax(dim=-1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_masked_argmax(cuda, dtype):
    from whisperdrz_amd import masked_argmax

    rows, V = 64, 51866
    g = torch.Generator(device=cuda).manual_seed(3)
    logits = (4.0 * torch.randn(rows, V, generator=g, device=cuda)).to(dtype)
    logits[5] = torch.round(logits[5].float()).to(dtype)  # many ties: lowest index wins
    blocked = torch.rand(rows, V, generator=g, device=cuda) < 0.3
    blocked[7] = True  # every token blocked
    penalty = torch.rand(rows, V, generator=g, device=cuda) < 0.01
    # the argmax of some rows is a penalised token (positive and negative maxima)
    top = logits.float().argmax(dim=-1)
    penalty[torch.arange(0, rows, 3, device=cuda), top[0::3]] = True
    logits[9] = -logits[9].abs()
    # NaN logits: torch.argmax takes a NaN as the maximum, so does the kernel
    logits[11, 1234] = float("nan")
    logits[12, 60] = float("nan")
    logits[12, 50] = float("nan")
    logits[13] = float("nan")
    print(f"masked_argmax {dtype}", flush=True)
    for b, p in [(blocked, penalty), (blocked, None), (None, penalty), (None, None)]:
        got = masked_argmax(logits, b, p)
        want = _reference_sampling(logits, b, p)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (got != want).nonzero()[:5].tolist()
