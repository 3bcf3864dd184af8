"""GPU parity of the fused MLP input projection (whisperdrz_amd.linear_gelu, wdrz_linear) with the
reference's two modules, Linear(n_state, 4 n_state) then nn.GELU() (src/whisperdrz/model.py:388-391),
on the same GPU tensors.

The fp32 reference is ``round16(gelu(round16(x W^T + b)))`` with the product in fp32, which is
what both the kernel and torch's 16-bit modules compute up to the order of the K-sum. Bar: within
two units in the last place of the 16-bit result (one for each rounding a different sum order can
flip) plus 2^-10 absolute (GELU's flat region near -0.75), with at least 97% of the elements
bit-identical to the fp32 reference; against torch's own 16-bit modules the same bar.

linear_partials (the MLP output projection split along K, wdrz_linear_partials): each fp32
partial against the float64 product of its K slice, within 1e-5 of the sum of |x_k w_k| (fp32
accumulation over at most a few thousand terms).
"""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _ulp16(t: torch.Tensor) -> torch.Tensor:
    bits = 7 if t.dtype == torch.bfloat16 else 10
    a = t.float().abs().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - bits)


def _check(y, ref, what):
    diff = (y.float() - ref.float()).abs()
    bound = 2 * _ulp16(ref) + 2.0 ** -10
    worst = (diff - bound).max().item()
    assert worst <= 0, f"{what}: max excess over the bound {worst}"
    same = (y == ref).float().mean().item()
    assert same >= 0.97, f"{what}: only {same:.4f} of the elements are bit-identical"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(1, 5120, 1280), (5, 5120, 1280), (64, 5120, 1280), (65, 2048, 512),
                                   (130, 40, 128), (3, 8, 384)])
@pytest.mark.parametrize("gelu", [True, False])
def test_linear_gelu(cuda, dtype, M, N, K, gelu):
    from whisperdrz_amd import linear_gelu

    print(f"linear {dtype} M={M} N={N} K={K} gelu={gelu}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(M * 7 + N + K)
    lin = torch.nn.Linear(K, N).to(cuda, dtype)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g, device=cuda) / K ** 0.5)
        lin.bias.copy_(0.5 * torch.randn(N, generator=g, device=cuda))
    x = torch.randn(M, K, generator=g, device=cuda).to(dtype)
    y = linear_gelu(x, lin, gelu)
    pre = (x.float() @ lin.weight.float().T + lin.bias.float()).to(dtype)
    ref = F.gelu(pre.float()).to(dtype) if gelu else pre
    with torch.no_grad():
        mod = F.gelu(lin(x)) if gelu else lin(x)
    torch.cuda.synchronize()
    _check(y, ref, "vs fp32 reference")
    _check(y, mod, "vs torch modules")


def test_linear_strided_rows_and_no_bias(cuda):
    """x rows taken from a wider buffer (a view, row stride > K) and a Linear without bias."""
    from whisperdrz_amd import linear_gelu

    dtype = torch.bfloat16
    g = torch.Generator(device=cuda).manual_seed(3)
    big = torch.randn(4, 2, 10, 512 + 64, generator=g, device=cuda).to(dtype)
    x = big[:, 1, :, :512]  # [4, 10, 512], rows of stride 576
    lin = torch.nn.Linear(512, 1024, bias=False).to(cuda, dtype)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(1024, 512, generator=g, device=cuda) / 512 ** 0.5)
    # a view with non-uniform outer strides is not a row matrix: refused, then the contiguous copy works
    with pytest.raises(ValueError):
        linear_gelu(x, lin)
    xs = big[:, 1, 3, :512]  # [4, 512], row stride 2*10*576
    y = linear_gelu(xs, lin)
    ref = F.gelu((xs.float() @ lin.weight.float().T).to(dtype).float()).to(dtype)
    torch.cuda.synchronize()
    _check(y, ref, "strided rows")


def test_linear_zero_rows_and_errors(cuda):
    from whisperdrz_amd import linear_gelu, _lib

    lin = torch.nn.Linear(128, 32).to(cuda, torch.bfloat16)
    y = linear_gelu(torch.empty(0, 128, device=cuda, dtype=torch.bfloat16), lin)
    assert y.shape == (0, 32)
    with pytest.raises(TypeError):
        linear_gelu(torch.randn(2, 64, device=cuda), lin)  # fp32 activations
    bad = torch.nn.Linear(96, 32).to(cuda, torch.bfloat16)  # K % 128 != 0
    with pytest.raises(NotImplementedError, match="multiple of 128"):
        linear_gelu(torch.randn(2, 96, device=cuda, dtype=torch.bfloat16), bad)
    lib = _lib.load()
    assert lib.wdrz_linear(_lib.WDRZ_BF16, None, 64, None, 64, None, None, 32, 1, 32, 128, 1, None) == _lib.WDRZ_EINVAL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K,n_split", [(64, 1280, 5120, 4), (1, 1280, 5120, 4), (5, 1280, 5120, 2),
                                           (65, 1024, 4096, 4), (130, 40, 1024, 2), (3, 8, 512, 4)])
def test_linear_partials(cuda, dtype, M, N, K, n_split):
    from whisperdrz_amd import linear_partials

    print(f"linear_partials {dtype} M={M} N={N} K={K} n_split={n_split}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(M * 3 + N + K + n_split)
    lin = torch.nn.Linear(K, N).to(cuda, dtype)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g, device=cuda) / K ** 0.5)
    x = torch.randn(M, K, generator=g, device=cuda).to(dtype)
    part = linear_partials(x, lin, n_split)
    torch.cuda.synchronize()
    assert part.dtype == torch.float32 and tuple(part.shape) == (n_split, M, N)
    kc = K // n_split
    w = lin.weight.double()
    for z in range(n_split):
        xs, ws = x[:, z * kc:(z + 1) * kc].double(), w[:, z * kc:(z + 1) * kc]
        ref = xs @ ws.T
        scale = xs.abs() @ ws.abs().T
        err = (part[z].double() - ref).abs()
        assert torch.all(err <= 1e-5 * scale + 1e-30), f"split {z}: max error {float(err.max())}"


def test_linear_partials_errors(cuda):
    from whisperdrz_amd import linear_partials

    lin = torch.nn.Linear(1000, 64).to(cuda, torch.bfloat16)
    x = torch.randn(4, 1000, device=cuda).to(torch.bfloat16)
    with pytest.raises(NotImplementedError, match="multiple of 128"):
        linear_partials(x, lin, 4)  # K = 1000
    lin2 = torch.nn.Linear(1024, 64).to(cuda, torch.bfloat16)
    x2 = torch.randn(4, 1024, device=cuda).to(torch.bfloat16)
    with pytest.raises(NotImplementedError, match="n_split 3"):
        linear_partials(x2, lin2, 3)

