"""GPU parity of the DTW alignment prep (wdrz_dtw_prep via whisperdrz_amd.dtw) against the
float64 oracle restating _dtw_prep_batch (src/whisperdrz/dtw_align.py:700-753).

Tolerance: fp32 contract, max |diff| <= 1e-5 * max |ref| over the finite entries; NaN exactly
where the reference has NaN (a batch row with cap 0 or length 0). The full bench shape is
checked against the reference's own op sequence run with torch fp32 ops on the GPU.
"""
import numpy as np
import pytest
import torch

from oracle.dtw_oracle import dtw_prep_ref, dtw_prep_torch

pytestmark = pytest.mark.gpu

TOL_REL = 1e-5


def _scores(shape, seed, scale=2.5):
    g = torch.Generator().manual_seed(seed)
    return scale * torch.randn(*shape, generator=g, dtype=torch.float32)


def _check(got: torch.Tensor, ref: np.ndarray, what: str):
    got = got.detach().cpu().numpy().astype(np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    nan_ref = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan_ref), f"{what}: NaN pattern differs"
    fin = ~nan_ref
    if fin.any():
        err = float(np.max(np.abs(got[fin] - ref[fin])))
        bound = TOL_REL * float(np.max(np.abs(ref[fin])))
        assert err <= bound, f"{what}: max|diff|={err:.3e} > {bound:.3e}"


def _run(cuda, w, lens, caps, width, what):
    from whisperdrz_amd import dtw_prep

    print(what, flush=True)
    out = dtw_prep(w.to(cuda), lens, caps, width)
    torch.cuda.synchronize()
    _check(out, dtw_prep_ref(w.numpy(), lens, caps, width), what)
    return out


@pytest.mark.parametrize("A", [203, 200])  # rows unaligned (column-strip kernels) / aligned (whole rows)
@pytest.mark.parametrize("width", [1, 3, 5, 7, 9, 15])
def test_widths(cuda, width, A):
    B, H, T = 3, 4, 37
    w = _scores((B, H, T, A), 10 + width + A)
    _run(cuda, w, [37, 20, 5], [A, 150, 61], width, f"dtw width={width} A={A}")


@pytest.mark.parametrize("B,H,T,A,lens,caps", [
    (1, 1, 1, 5, [1], [5]),                    # single row, narrow
    (2, 10, 64, 1500, [64, 33], [1500, 1499]),  # whole window, cap just short of A
    (2, 3, 130, 257, [200, 130], [257, 3]),     # length beyond T (divides by the length), cap 3
    (3, 2, 17, 130, [17, 9, 12], [130, 127, 66]),
    (2, 2, 448, 96, [448, 300], [96, 50]),      # the full text context
    # fused row/column pass (rows 16-byte aligned, A <= 2048): 1, 2 and 3 row chunks of 64,
    # every register width, a length beyond T
    (2, 3, 70, 1000, [70, 65], [1000, 999]),
    (2, 2, 130, 512, [130, 129], [511, 512]),
    (2, 2, 100, 1500, [150, 100], [1500, 1497]),
    (1, 2, 64, 2048, [64], [2047]),
    (1, 2, 20, 2100, [20], [2100]),             # A > 2048: separate row and column passes
    # width 7 with A >= 256 (250-column wavefront segments; reflected columns at both ends of
    # the first and last segment): one segment that is both, a last segment of 3 columns,
    # T not a multiple of the 4 rows per wavefront
    (2, 3, 21, 256, [21, 7], [256, 200]),
    (1, 2, 9, 260, [9], [260]),
    (2, 2, 13, 503, [13, 13], [503, 251]),
    (1, 2, 6, 1504, [6], [1504]),
    (1, 16, 5, 300, [5], [300]),                # the most heads this path unrolls
    (1, 17, 5, 300, [5], [300]),                # one more: the column-strip filter
])
def test_shapes(cuda, B, H, T, A, lens, caps):
    w = _scores((B, H, T, A), B * 1000 + T + A)
    _run(cuda, w, lens, caps, 7, f"dtw B={B} H={H} T={T} A={A} lens={lens} caps={caps}")


def test_degenerate_rows_are_nan(cuda):
    w = _scores((3, 2, 9, 40), 5)
    out = _run(cuda, w, [9, 0, 5], [40, 30, 0], 7, "dtw degenerate cap/len")
    assert torch.isnan(out[1]).all() and torch.isnan(out[2]).all()


def test_short_audio_axis_skips_filter(cuda):
    # T_audio <= width // 2: the reference returns the input of the filter unchanged
    w = _scores((2, 3, 6, 3), 6)
    _run(cuda, w, [6, 4], [3, 2], 7, "dtw A=3 width=7")


def test_strided_scores(cuda):
    # a view whose rows are longer than T_audio (strides stay multiples of 4 elements)
    base = _scores((2, 3, 21, 72), 7)
    w = base[:, :, :, :65]
    from whisperdrz_amd import dtw_prep

    print("dtw strided view", flush=True)
    out = dtw_prep(base.to(cuda)[:, :, :, :65], [21, 10], [65, 40], 7)
    torch.cuda.synchronize()
    _check(out, dtw_prep_ref(w.numpy(), [21, 10], [65, 40], 7), "dtw strided view")


def test_strided_unaligned_rows_width7(cuda):
    # rows that start 4 bytes past a 16-byte boundary and a row pitch that is not a multiple
    # of 4: the separate row / column statistics passes, then the segment filter
    base = _scores((2, 3, 11, 301), 9)
    w = base[:, :, :, 1:290]
    from whisperdrz_amd import dtw_prep

    print("dtw strided unaligned width 7", flush=True)
    out = dtw_prep(base.to(cuda)[:, :, :, 1:290], [11, 6], [289, 270], 7)
    torch.cuda.synchronize()
    _check(out, dtw_prep_ref(w.numpy(), [11, 6], [289, 270], 7), "dtw strided unaligned width 7")


def test_batch_returns_host_array_and_is_deterministic(cuda):
    from whisperdrz_amd import dtw_prep, dtw_prep_batch

    w = _scores((4, 10, 100, 1500), 8).to(cuda)
    lens, caps = [100, 80, 60, 99], [1500, 1200, 700, 1499]
    print("dtw batch host copy", flush=True)
    a = dtw_prep(w, lens, caps).cpu().numpy()
    b = dtw_prep_batch(w, lens, caps)
    assert isinstance(b, np.ndarray) and b.shape == (4, 100, 1500) and b.dtype == np.float32
    np.testing.assert_array_equal(a, b)


def test_bench_shape_matches_torch_ops(cuda):
    # The bench workload (16 chunks x 10 alignment heads x 448 text rows x 1500 audio columns)
    # against the reference's op sequence in torch fp32 on the same GPU.
    from whisperdrz_amd import dtw_prep

    B, H, T, A = 16, 10, 448, 1500
    g = torch.Generator(device=cuda).manual_seed(11)
    w = 2.5 * torch.randn((B, H, T, A), generator=g, device=cuda)
    rng = np.random.default_rng(11)
    lens = [int(x) for x in rng.integers(T // 2, T + 1, B)]
    caps = [int(x) for x in rng.integers(A // 2, A + 1, B)]
    caps[0] = A
    print("dtw bench shape vs torch ops", flush=True)
    out = dtw_prep(w, lens, caps)
    ref = dtw_prep_torch(w, lens, caps)  # torch ops on the GPU tensor (fp32)
    torch.cuda.synchronize()
    err = (out - ref).abs().max().item()
    assert err <= 1e-4 * ref.abs().max().item(), err


# ---- CrossAttnCapture.compute_attention (dtw_align.py:553-586) ----------------------------


def _captures(B, T, A, n_layers, n_heads, dtype, seed):
    """Per-layer query / key projections as the capture hooks hold them ([B, T, n_heads*64])."""
    g = torch.Generator().manual_seed(seed)
    q_out = [torch.randn(B, T, n_heads * 64, generator=g).to(dtype) for _ in range(n_layers)]
    k_out = [torch.randn(B, A, n_heads * 64, generator=g).to(dtype) for _ in range(n_layers)]
    return q_out, k_out


def _qk_ref(q_out, k_out, head_mask, n_heads):
    from oracle.dtw_oracle import compute_attention_ref

    sel = head_mask.nonzero().tolist()
    qh = np.stack([q_out[l].float().view(q_out[l].shape[0], q_out[l].shape[1], n_heads, 64)[:, :, h].numpy()
                   for l, h in sel])
    kh = np.stack([k_out[l].float().view(k_out[l].shape[0], k_out[l].shape[1], n_heads, 64)[:, :, h].numpy()
                   for l, h in sel])
    return compute_attention_ref(qh, kh, 64)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,A", [(2, 37, 1500), (3, 64, 203), (1, 5, 70)])
def test_compute_attention(cuda, dtype, B, T, A):
    from whisperdrz_amd import compute_attention

    n_layers, n_heads = 6, 20
    q_out, k_out = _captures(B, T, A, n_layers, n_heads, dtype, seed=B * 100 + T + A)
    head_mask = torch.zeros(n_layers, n_heads, dtype=torch.bool)
    for l, h in [(1, 0), (1, 17), (3, 5), (4, 19), (5, 2), (5, 11)]:
        head_mask[l, h] = True
    print(f"compute_attention {dtype} B={B} T={T} A={A}", flush=True)
    got = compute_attention([q.to(cuda) for q in q_out], [k.to(cuda) for k in k_out], head_mask)
    torch.cuda.synchronize()
    ref = _qk_ref(q_out, k_out, head_mask, n_heads)
    if B == 1:
        assert got.dim() == 3  # the reference drops the batch axis for one chunk
        ref = ref[0]
    _check(got, ref, f"compute_attention {dtype} B={B} T={T} A={A}")


def test_compute_attention_mixed_layouts_and_prep_chain(cuda):
    # one layer's projection is a column slice of a wider tensor (other strides): the heads are
    # given one layout; then the scores go through the prep, against the oracle chain
    from whisperdrz_amd import compute_attention, dtw_prep
    from oracle.dtw_oracle import dtw_prep_ref

    B, T, A, n_layers, n_heads = 2, 40, 1500, 3, 20
    q_out, k_out = _captures(B, T, A, n_layers, n_heads, torch.bfloat16, seed=77)
    wide = torch.randn(B, T, 2 * n_heads * 64, generator=torch.Generator().manual_seed(78)).to(torch.bfloat16)
    q_out[2] = wide[:, :, : n_heads * 64]
    head_mask = torch.zeros(n_layers, n_heads, dtype=torch.bool)
    head_mask[0, 3] = head_mask[2, 7] = head_mask[2, 8] = True
    print("compute_attention mixed layouts + prep", flush=True)
    dev_q = [q.to(cuda) if i != 2 else wide.to(cuda)[:, :, : n_heads * 64] for i, q in enumerate(q_out)]
    got = compute_attention(dev_q, [k.to(cuda) for k in k_out], head_mask)
    ref = _qk_ref([q.contiguous() for q in q_out], k_out, head_mask, n_heads)
    _check(got, ref, "compute_attention mixed layouts")
    lens, caps = [40, 23], [1500, 1211]
    out = dtw_prep(got, lens, caps)
    torch.cuda.synchronize()
    _check(out, dtw_prep_ref(got.cpu().numpy(), lens, caps, 7), "prep of computed scores")


def test_compute_attention_rejects(cuda):
    from whisperdrz_amd import compute_attention

    q_out, k_out = _captures(1, 4, 8, 1, 20, torch.float32, seed=1)
    mask = torch.zeros(1, 20, dtype=torch.bool)
    with pytest.raises(ValueError):
        compute_attention([q_out[0].to(cuda)], [k_out[0].to(cuda)], mask)  # no heads selected
    mask[0, 0] = True
    with pytest.raises(TypeError):
        compute_attention([q_out[0].to(cuda)], [k_out[0].to(cuda)], mask)  # fp32 projections


# ---- fused: compute_attention + prep without the score tensor (dtw_align.py:1184-1197) ------
# Against the float64 oracle chain dtw_prep_ref(compute_attention_ref(...)): the scores carry
# fp32 accumulation error (about 1e-7 of |S|), which the column normalisation can amplify, so
# the bound is 1e-4 * max |ref|; against the two-kernel GPU chain (the same fp32 products,
# summed in another order) the same bound holds.
FUSED_TOL_REL = 1e-4


def _check_fused(got, ref, what):
    got = got.detach().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    nan_ref = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan_ref), f"{what}: NaN pattern differs"
    fin = ~nan_ref
    if fin.any():
        err = float(np.max(np.abs(got[fin] - ref[fin])))
        bound = FUSED_TOL_REL * float(np.max(np.abs(ref[fin])))
        assert err <= bound, f"{what}: max|diff|={err:.3e} > {bound:.3e}"


def _mask(n_layers, n_heads, pairs):
    m = torch.zeros(n_layers, n_heads, dtype=torch.bool)
    for l, h in pairs:
        m[l, h] = True
    return m


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,A,lens,caps,width", [
    (2, 37, 1500, [37, 20], [1500, 751], 7),     # Whisper's audio axis, ragged text / caps
    (3, 64, 203, [64, 1, 30], [203, 100, 0], 7),  # cap 0 -> NaN row; one valid text row
    (1, 5, 70, [5], [70], 3),
    (2, 130, 257, [200, 130], [257, 3], 5),      # length beyond T; cap 3
    (1, 17, 5, [17], [5], 7),                    # A = 5: reflect halo on both sides at once
    (1, 9, 3, [9], [3], 7),                      # A <= width // 2: unfiltered
    (1, 33, 1536, [33], [1536], 15),             # the largest audio axis, widest filter
    (2, 20, 96, [0, 20], [96, 96], 1),           # length 0 -> NaN row; no filter
])
def test_attention_prep_fused(cuda, dtype, B, T, A, lens, caps, width):
    from whisperdrz_amd import dtw_attention_prep

    n_layers, n_heads = 6, 20
    q_out, k_out = _captures(B, T, A, n_layers, n_heads, dtype, seed=7 * B + T + A + width)
    head_mask = _mask(n_layers, n_heads, [(1, 0), (1, 17), (3, 5), (4, 19), (5, 2), (5, 11)])
    what = f"dtw_attention_prep {dtype} B={B} T={T} A={A} width={width}"
    print(what, flush=True)
    got = dtw_attention_prep([q.to(cuda) for q in q_out], [k.to(cuda) for k in k_out], head_mask, lens, caps,
                             width)
    torch.cuda.synchronize()
    ref = dtw_prep_ref(_qk_ref(q_out, k_out, head_mask, n_heads), lens, caps, width)
    _check_fused(got, ref, what)


@pytest.mark.parametrize("heads,B,T,A,lens,caps,width", [
    ([(0, 4)], 1, 1, 1500, [1], [1500], 7),              # one head, one text row (n = 1: zero variance)
    ([(0, 1), (2, 9), (3, 3)], 2, 33, 1500, [33, 2], [900, 1500], 7),  # odd head count, tiny length
    ([(1, 0), (1, 1)], 3, 64, 17, [64, 64, 10], [17, 1, 16], 3),       # A = 17 (one key past a tile)
])
def test_attention_prep_fused_heads_and_edges(cuda, heads, B, T, A, lens, caps, width):
    from whisperdrz_amd import dtw_attention_prep

    n_layers, n_heads = 4, 20
    q_out, k_out = _captures(B, T, A, n_layers, n_heads, torch.float16, seed=1000 + T + A)
    head_mask = _mask(n_layers, n_heads, heads)
    what = f"dtw_attention_prep H={len(heads)} B={B} T={T} A={A} width={width}"
    print(what, flush=True)
    got = dtw_attention_prep([q.to(cuda) for q in q_out], [k.to(cuda) for k in k_out], head_mask, lens, caps,
                             width)
    torch.cuda.synchronize()
    ref = dtw_prep_ref(_qk_ref(q_out, k_out, head_mask, n_heads), lens, caps, width)
    _check_fused(got, ref, what)


def test_attention_prep_fused_many_heads_and_layouts(cuda):
    # 32 heads (the most the entry takes), one projection a column slice of a wider tensor
    from whisperdrz_amd import dtw_attention_prep

    B, T, A, n_layers, n_heads = 2, 48, 1500, 2, 20
    q_out, k_out = _captures(B, T, A, n_layers, n_heads, torch.bfloat16, seed=91)
    wide = torch.randn(B, T, 2 * n_heads * 64, generator=torch.Generator().manual_seed(92)).to(torch.bfloat16)
    q_out[1] = wide[:, :, : n_heads * 64]
    head_mask = _mask(n_layers, n_heads, [(l, h) for l in range(2) for h in range(16)])
    lens, caps = [48, 31], [1500, 1100]
    print("dtw_attention_prep 32 heads, mixed layouts", flush=True)
    dev_q = [q_out[0].to(cuda), wide.to(cuda)[:, :, : n_heads * 64]]
    got = dtw_attention_prep(dev_q, [k.to(cuda) for k in k_out], head_mask, lens, caps)
    torch.cuda.synchronize()
    ref = dtw_prep_ref(_qk_ref([q.contiguous() for q in q_out], k_out, head_mask, n_heads), lens, caps, 7)
    _check_fused(got, ref, "dtw_attention_prep 32 heads")


def test_attention_prep_fused_bench_shape_matches_chain(cuda):
    # The bench workload: 16 chunks x 448 text rows x 1500 audio columns, large-v3's 10
    # alignment heads, against compute_attention + dtw_prep on the same GPU, and repeatable.
    from whisperdrz_amd import compute_attention, dtw_attention_prep, dtw_prep

    B, T, A, n_layers, n_heads = 16, 448, 1500, 32, 20
    heads = [(7, 0), (10, 17), (12, 18), (13, 12), (16, 1), (17, 14), (19, 11), (21, 4), (24, 1), (25, 6)]
    g = torch.Generator(device=cuda).manual_seed(5)
    used = {l for l, _ in heads}
    q_out = [torch.randn(B, T, n_heads * 64, generator=g, device=cuda).to(torch.bfloat16) if l in used else None
             for l in range(n_layers)]
    k_out = [torch.randn(B, A, n_heads * 64, generator=g, device=cuda).to(torch.bfloat16) if l in used else None
             for l in range(n_layers)]
    head_mask = _mask(n_layers, n_heads, heads)
    rng = np.random.default_rng(5)
    lens = [int(x) for x in rng.integers(T // 2, T + 1, B)]
    caps = [int(x) for x in rng.integers(A // 2, A + 1, B)]
    caps[0] = A
    print("dtw_attention_prep bench shape vs chain", flush=True)
    got = dtw_attention_prep(q_out, k_out, head_mask, lens, caps)
    again = dtw_attention_prep(q_out, k_out, head_mask, lens, caps)
    chain = dtw_prep(compute_attention(q_out, k_out, head_mask), lens, caps)
    torch.cuda.synchronize()
    assert torch.equal(got, again)
    err = (got - chain).abs().max().item()
    assert err <= FUSED_TOL_REL * chain.abs().max().item(), err


def test_attention_prep_fused_rejects(cuda):
    from whisperdrz_amd import dtw_attention_prep

    q_out, k_out = _captures(1, 4, 1600, 1, 20, torch.bfloat16, seed=3)
    mask = _mask(1, 20, [(0, 0)])
    with pytest.raises(NotImplementedError):  # audio axis beyond 1536
        dtw_attention_prep([q_out[0].to(cuda)], [k_out[0].to(cuda)], mask, [4], [1600])
    with pytest.raises(ValueError):
        dtw_attention_prep([q_out[0].to(cuda)], [k_out[0].to(cuda)], mask, [4, 4], [8, 8])  # B mismatch


# ---- median_filter (dtw_align.py:156-167), standalone ----------------------------------------


@pytest.mark.parametrize("width", [1, 3, 5, 7, 9, 11, 13, 15])
@pytest.mark.parametrize("shape", [(3, 4, 1500), (2, 2049), (7, 8), (1, 5)])
def test_median_filter_matches_oracle(cuda, width, shape):
    from oracle.dtw_oracle import median_filter_ref
    from whisperdrz_amd import median_filter

    x = _scores(shape, seed=width * 100 + shape[-1])
    print(f"median_filter width={width} shape={shape}", flush=True)
    got = median_filter(x.to(cuda), width)
    torch.cuda.synchronize()
    assert got.shape == x.shape and got.dtype == x.dtype
    np.testing.assert_array_equal(got.cpu().numpy(), median_filter_ref(x.numpy(), width))  # a selection: exact


def test_median_filter_strided_bf16_and_rejects(cuda):
    from oracle.dtw_oracle import median_filter_ref
    from whisperdrz_amd import median_filter

    wide = _scores((6, 2 * 300), seed=5).to(cuda)
    x = wide[:, ::2]  # last stride 2
    print("median_filter strided / bf16 / rejects", flush=True)
    np.testing.assert_array_equal(median_filter(x, 7).cpu().numpy(), median_filter_ref(x.cpu().numpy(), 7))
    xb = _scores((4, 100), seed=6).to(torch.bfloat16)
    got = median_filter(xb.to(cuda), 5)
    assert got.dtype == torch.bfloat16
    np.testing.assert_array_equal(got.float().cpu().numpy(), median_filter_ref(xb.float().numpy(), 5))
    with pytest.raises(ValueError):
        median_filter(x, 4)  # even width: the reference's own reshape fails
    with pytest.raises(NotImplementedError):
        median_filter(x, 17)
