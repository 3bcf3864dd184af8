"""The C-ABI library: it loads (no GPU needed), exports every function include/wdrz_attn.h
declares, and rejects bad arguments on the host with a code and a message before any launch."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wdrz_attn.h")


@pytest.fixture(scope="module")
def lib():
    from whisperdrz_amd import _lib

    if not _lib.LIB_PATH.exists():
        from whisperdrz_amd.build import build_library

        build_library()
    return _lib.load()


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\*\s]+?\b(wdrz_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for n in ("wdrz_attn_fwd", "wdrz_attn_kvcache", "wdrz_attn_kvcache_workspace_size", "wdrz_last_error",
              "wdrz_abi_version"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    from whisperdrz_amd import _lib

    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in wdrz_attn.h but not exported"
    assert set(declared_functions()) == set(_lib.EXPORTED_SYMBOLS)


def test_abi_version(lib):
    from whisperdrz_amd import _lib

    assert lib.wdrz_abi_version() == _lib.ABI_VERSION


def test_build_id_matches_the_tree(lib):
    """The loaded library was built from these sources (load() refuses any other)."""
    from whisperdrz_amd.build import source_hash

    assert lib.wdrz_build_id().decode() == source_hash()
    assert len(source_hash()) == 16


def test_workspace_size_plan(lib):
    # many rows: one workgroup per row, no workspace; few rows: split keys, workspace needed
    assert lib.wdrz_attn_kvcache_workspace_size(64, 1, 20, 64, 448) == 0
    assert lib.wdrz_attn_kvcache_workspace_size(64, 1, 20, 64, 1500) == 0
    small = lib.wdrz_attn_kvcache_workspace_size(1, 1, 20, 64, 1500)
    assert small > 0 and small % 4 == 0
    assert lib.wdrz_attn_kvcache_workspace_size(1, 5, 20, 64, 1500) > small
    assert lib.wdrz_attn_kvcache_workspace_size(0, 1, 20, 64, 448) == 0
    # 40+ query rows never split their keys (the prefill kernel's route): no workspace, however
    # few rows there are
    assert lib.wdrz_attn_kvcache_workspace_size(1, 39, 20, 64, 448) > 0
    assert lib.wdrz_attn_kvcache_workspace_size(1, 40, 20, 64, 448) == 0
    assert lib.wdrz_attn_kvcache_workspace_size(1, 224, 20, 64, 1500) == 0


def _strides(*s):
    return (ctypes.c_int64 * 4)(*s)


FAKE = 0x10000  # 16-byte-aligned non-null pointer value; validation fails before any use


def call_fwd(lib, **over):
    args = dict(dtype=2, q=FAKE, k=FAKE, v=FAKE, o=FAKE, B=1, H=2, Lq=8, Lk=8, D=64,
                qs=_strides(1024, 512, 64, 1), ks=_strides(1024, 512, 64, 1), vs=_strides(1024, 512, 64, 1),
                os_=_strides(1024, 512, 64, 1), scale=0.125, causal=0)
    args.update(over)
    return lib.wdrz_attn_fwd(args["dtype"], args["q"], args["k"], args["v"], args["o"], args["B"], args["H"],
                             args["Lq"], args["Lk"], args["D"], args["qs"], args["ks"], args["vs"], args["os_"],
                             args["scale"], args["causal"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(dtype=7), 1, "dtype"),
    (dict(D=32), 2, "head_dim"),
    (dict(q=None), 1, "q is NULL"),
    (dict(k=FAKE + 2), 1, "not 16-byte aligned"),
    (dict(Lk=0), 1, "bad sizes"),
    (dict(scale=-1.0), 1, "scale"),
    (dict(qs=_strides(1024, 512, 64, 2)), 1, "head_dim stride"),
    (dict(vs=_strides(1024, 512, 60, 1)), 1, "not 16-byte aligned"),
])
def test_fwd_rejects_bad_arguments(lib, over, code, msg):
    assert call_fwd(lib, **over) == code
    assert msg in lib.wdrz_last_error().decode()


def test_fwd_empty_batch_is_a_no_op(lib):
    assert call_fwd(lib, B=0) == 0
    assert lib.wdrz_last_error().decode() == ""


def call_kv(lib, **over):
    s = _strides(1024, 1024, 64, 1)
    args = dict(dtype=2, q=FAKE, kc=FAKE, vc=FAKE, kn=None, vn=None, seqlens=None, bidx=None, o=FAKE, B=2, sq=1,
                H=2, D=64, n_slots=4, Lmax=16, ws=None, ws_bytes=0, scale=0.125)
    args.update(over)
    return lib.wdrz_attn_kvcache(args["dtype"], args["q"], args["kc"], args["vc"], args["kn"], args["vn"],
                                 args["seqlens"], args["bidx"], args["o"], args["B"], args["sq"], args["H"], args["D"],
                                 args["n_slots"], args["Lmax"], s, s, s, s, s, s, args["scale"], 1, args["ws"],
                                 args["ws_bytes"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(kn=FAKE), 1, "k and v must be given together"),
    (dict(kn=FAKE, vn=FAKE), 1, "cache_seqlens is required"),
    (dict(kn=FAKE, vn=FAKE, seqlens=FAKE, sq=40), 1, "exceeds cache length"),
    (dict(D=128), 2, "head_dim"),
    (dict(kc=None), 1, "k_cache is NULL"),
    (dict(B=1, Lmax=1500), 4, "workspace"),
    (dict(scale=float("nan")), 1, "softmax_scale"),
])
def test_kvcache_rejects_bad_arguments(lib, over, code, msg):
    assert call_kv(lib, **over) == code
    assert msg in lib.wdrz_last_error().decode()


def call_dtw(lib, **over):
    args = dict(w=FAKE, ws_=_strides(4 * 16 * 64, 16 * 64, 64, 1), lens=FAKE, caps=FAKE, out=FAKE,
                os_=(ctypes.c_int64 * 3)(16 * 60, 60, 1), B=1, H=4, T=16, A=64, C=60, width=7, work=None,
                work_bytes=0)
    args.update(over)
    return lib.wdrz_dtw_prep(args["w"], args["ws_"], args["lens"], args["caps"], args["out"], args["os_"], args["B"],
                             args["H"], args["T"], args["A"], args["C"], args["width"], args["work"],
                             args["work_bytes"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(width=4), 1, "must be 1 or odd"),
    (dict(width=0), 1, "must be 1 or odd"),
    (dict(width=17), 2, "exceeds the supported 15"),
    (dict(T=513), 2, "exceed the supported 512"),
    (dict(C=65), 1, "exceeds A"),
    (dict(H=0), 1, "bad sizes"),
    (dict(w=None), 1, "weights is NULL"),
    (dict(ws_=_strides(4 * 16 * 64, 16 * 64, 64, 2)), 1, "last stride"),
    (dict(lens=None), 1, "actual_lens"),
    (dict(), 4, "workspace"),
    (dict(work=FAKE + 16, work_bytes=1 << 20), 1, "256-byte aligned"),
])
def test_dtw_prep_rejects_bad_arguments(lib, over, code, msg):
    assert call_dtw(lib, **over) == code
    assert msg in lib.wdrz_last_error().decode()


def test_dtw_prep_empty_is_a_no_op(lib):
    assert call_dtw(lib, B=0) == 0
    assert call_dtw(lib, C=0) == 0
    assert call_dtw(lib, T=0) == 0


def test_dtw_workspace_size(lib):
    B, H, T, A = 16, 10, 448, 1500
    n = lib.wdrz_dtw_prep_workspace_size(B, H, T, A)
    # row stats + column stats + column partials of the row chunks (as many chunks as keep
    # B*H*chunks <= 768: 4 chunks of 112 rows here), each 256-byte aligned
    assert n == 8 * B * H * (T + A + 4 * A)
    assert lib.wdrz_dtw_prep_workspace_size(0, H, T, A) == 0


def call_qk(lib, **over):
    H = over.pop("H", 2)
    ptrs = (ctypes.c_void_p * max(H, 1))(*([FAKE] * max(H, 1)))
    args = dict(dtype=2, q=ptrs, qs=(ctypes.c_int64 * 3)(40 * 1280, 1280, 1), k=ptrs,
                ks=(ctypes.c_int64 * 3)(1500 * 1280, 1280, 1), out=FAKE,
                os_=_strides(H * 40 * 1500, 40 * 1500, 1500, 1), B=1, T=40, A=1500, D=64, scale=64 ** -0.25)
    args.update(over)
    return lib.wdrz_dtw_qk(args["dtype"], args["q"], args["qs"], args["k"], args["ks"], args["out"], args["os_"],
                           args["B"], H, args["T"], args["A"], args["D"], args["scale"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(dtype=0), 2, "only WDRZ_BF16 / WDRZ_F16"),
    (dict(dtype=9), 1, "only WDRZ_BF16 / WDRZ_F16"),
    (dict(D=128), 2, "head_dim"),
    (dict(H=33), 2, "exceed the supported 32"),
    (dict(qs=(ctypes.c_int64 * 3)(40 * 1280, 1283, 1)), 1, "not 16-byte aligned"),
    (dict(ks=(ctypes.c_int64 * 3)(1500 * 1280, 1280, 2)), 1, "head_dim stride"),
    (dict(out=None), 1, "out is NULL"),
    (dict(scale=0.0), 1, "scale"),
])
def test_dtw_qk_rejects_bad_arguments(lib, over, code, msg):
    assert call_qk(lib, **over) == code
    assert msg in lib.wdrz_last_error().decode()


def test_dtw_qk_empty_is_a_no_op(lib):
    assert call_qk(lib, B=0) == 0


def call_attn_prep(lib, **over):
    H = over.pop("H", 2)
    ptrs = (ctypes.c_void_p * max(H, 1))(*([FAKE] * max(H, 1)))
    args = dict(dtype=2, q=ptrs, qs=(ctypes.c_int64 * 3)(40 * 1280, 1280, 1), k=ptrs,
                ks=(ctypes.c_int64 * 3)(1500 * 1280, 1280, 1), scale=64 ** -0.25, lens=FAKE, caps=FAKE, out=FAKE,
                os_=(ctypes.c_int64 * 3)(40 * 1500, 1500, 1), B=1, T=40, A=1500, D=64, C=1500, width=7,
                work=None, work_bytes=0)
    args.update(over)
    return lib.wdrz_dtw_attention_prep(args["dtype"], args["q"], args["qs"], args["k"], args["ks"], args["scale"],
                                       args["lens"], args["caps"], args["out"], args["os_"], args["B"], H,
                                       args["T"], args["A"], args["D"], args["C"], args["width"], args["work"],
                                       args["work_bytes"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(A=1537, C=1537), 2, "exceed the supported 1536"),
    (dict(dtype=0), 2, "only WDRZ_BF16 / WDRZ_F16"),
    (dict(D=128), 2, "head_dim"),
    (dict(H=33), 2, "exceed the supported 32"),
    (dict(scale=float("nan")), 1, "scale"),
    (dict(width=4), 1, "must be 1 or odd"),
    (dict(T=513), 2, "exceed the supported 512"),
    (dict(C=1501), 1, "exceeds A"),
    (dict(lens=None), 1, "actual_lens"),
    (dict(), 4, "workspace"),
])
def test_dtw_attention_prep_rejects_bad_arguments(lib, over, code, msg):
    assert call_attn_prep(lib, **over) == code
    assert msg in lib.wdrz_last_error().decode()


def test_dtw_attention_prep_empty_is_a_no_op(lib):
    assert call_attn_prep(lib, B=0) == 0
    assert call_attn_prep(lib, C=0) == 0


@pytest.mark.parametrize("over,code,msg", [
    (dict(n=200), 1, "reflect padding"),
    (dict(n_mels=129), 2, "exceeds the supported 128"),
    (dict(audio=None), 1, "is NULL"),
    (dict(), 4, "workspace"),
])
def test_log_mel_rejects_bad_arguments(lib, over, code, msg):
    args = dict(audio=FAKE, B=2, n=480000, stride=480000, out=FAKE, n_mels=128, frames=3000)
    args.update(over)
    os3 = (ctypes.c_int64 * 3)(args["n_mels"] * 3000, 3000, 1)
    rc = lib.wdrz_log_mel(args["audio"], args["B"], args["n"], args["stride"], args["out"], os3, args["n_mels"],
                          args["frames"], None, 0, None)
    assert rc == code
    assert msg in lib.wdrz_last_error().decode()


def call_fill(lib, **over):
    args = dict(dtype=2, k=FAKE, v=FAKE, ss=(ctypes.c_int64 * 3)(1500 * 2560, 2560, 64), kc=FAKE, vc=FAKE,
                cs=(ctypes.c_int64 * 3)(20 * 1500 * 64, 64, 1500 * 64), slots=None, B=16, T=1500, H=20, D=64,
                n_slots=64, Lmax=1500, start=0)
    args.update(over)
    return lib.wdrz_kv_fill(args["dtype"], args["k"], args["v"], args["ss"], args["kc"], args["vc"], args["cs"],
                            args["slots"], args["B"], args["T"], args["H"], args["D"], args["n_slots"],
                            args["Lmax"], args["start"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(dtype=0), 2, "only WDRZ_BF16 / WDRZ_F16"),
    (dict(D=128), 2, "head_dim"),
    (dict(start=1), 1, "exceed the cache length"),
    (dict(k=None), 1, "is NULL"),
    (dict(kc=FAKE + 8), 1, "16-byte aligned"),
    (dict(ss=(ctypes.c_int64 * 3)(1500 * 2560, 2561, 64)), 1, "16-byte aligned"),
    (dict(T=-1), 1, "bad sizes"),
])
def test_kv_fill_rejects_bad_arguments(lib, over, code, msg):
    assert call_fill(lib, **over) == code
    assert msg in lib.wdrz_last_error().decode()


def test_kv_fill_empty_is_a_no_op(lib):
    assert call_fill(lib, B=0) == 0
    assert call_fill(lib, T=0) == 0


@pytest.mark.parametrize("width,code,msg", [(4, 1, "must be 1 or odd"), (0, 1, "must be 1 or odd"),
                                            (17, 2, "exceeds the supported 15")])
def test_median_filter_rejects_bad_widths(lib, width, code, msg):
    assert lib.wdrz_median_filter(FAKE, 100, FAKE, 100, 4, 100, width, None) == code
    assert msg in lib.wdrz_last_error().decode()


def test_median_filter_rejects_short_strides_and_empty_is_a_no_op(lib):
    assert lib.wdrz_median_filter(FAKE, 50, FAKE, 100, 4, 100, 7, None) == 1
    assert "row strides" in lib.wdrz_last_error().decode()
    assert lib.wdrz_median_filter(FAKE, 100, FAKE, 100, 0, 100, 7, None) == 0


def call_linear(lib, **over):
    args = dict(dtype=2, x=FAKE, xs=1280, w=FAKE, ws=1280, b=FAKE, y=FAKE, ys=5120, M=64, N=5120, K=1280, act=1)
    args.update(over)
    return lib.wdrz_linear(args["dtype"], args["x"], args["xs"], args["w"], args["ws"], args["b"], args["y"],
                           args["ys"], args["M"], args["N"], args["K"], args["act"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(dtype=0), 2, "only WDRZ_BF16 / WDRZ_F16"),
    (dict(act=2), 1, "activation 2"),
    (dict(K=1216), 2, "multiple of 128"),
    (dict(N=5124), 2, "multiple of 128 and N=5124 of 8"),
    (dict(N=0), 1, "bad sizes"),
    (dict(w=None), 1, "is NULL"),
    (dict(y=FAKE + 8), 1, "16-byte aligned"),
    (dict(b=FAKE + 1), 1, "2-byte aligned"),
    (dict(xs=1000), 1, "shorter than the rows"),
    (dict(xs=1284), 1, "16-byte aligned"),
    (dict(M=65535 * 64 + 1), 2, "sizes too large"),
])
def test_linear_rejects_bad_arguments(lib, over, code, msg):
    assert call_linear(lib, **over) == code
    assert msg in lib.wdrz_last_error().decode()


def test_linear_zero_rows_is_a_no_op(lib):
    assert call_linear(lib, M=0, x=None, w=None, y=None) == 0


def call_linear_partials(lib, **over):
    args = dict(dtype=2, x=FAKE, xs=5120, w=FAKE, ws=5120, p=FAKE, M=64, N=1280, K=5120, ns=4)
    args.update(over)
    return lib.wdrz_linear_partials(args["dtype"], args["x"], args["xs"], args["w"], args["ws"], args["p"],
                                    args["M"], args["N"], args["K"], args["ns"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(dtype=0), 2, "only WDRZ_BF16 / WDRZ_F16"),
    (dict(ns=3), 2, "n_split 3 is not 2 or 4"),
    (dict(K=5120 - 128), 2, "multiple of 128 * n_split"),
    (dict(N=1284), 2, "N=1284 of 8"),
    (dict(M=-1), 1, "bad sizes"),
    (dict(p=None), 1, "partials is NULL"),
    (dict(p=FAKE + 4), 1, "16-byte aligned"),
    (dict(ws=4096), 1, "shorter than the rows"),
    (dict(xs=5124), 1, "16-byte aligned"),
])
def test_linear_partials_rejects_bad_arguments(lib, over, code, msg):
    assert call_linear_partials(lib, **over) == code
    assert msg in lib.wdrz_last_error().decode()


def test_linear_partials_zero_rows_is_a_no_op(lib):
    assert call_linear_partials(lib, M=0, x=None, w=None, p=None) == 0


def call_add_ln_partials(lib, **over):
    args = dict(dtype=2, x=FAKE, xs=1280, p=FAKE, ns=4, db=FAKE, w=FAKE, b=FAKE, y=FAKE, ys=1280, rows=64,
                n=1280, eps=1e-5)
    args.update(over)
    return lib.wdrz_add_layernorm_partials(args["dtype"], args["x"], args["xs"], args["p"], args["ns"], args["db"],
                                           args["w"], args["b"], args["y"], args["ys"], args["rows"], args["n"],
                                           args["eps"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(dtype=0), 2, "only WDRZ_BF16 / WDRZ_F16"),
    (dict(ns=8), 2, "n_split 8 is not 2 or 4"),
    (dict(n=1284), 1, "multiple of 8"),
    (dict(n=2048), 2, "exceeds the supported 1536"),
    (dict(eps=-1.0), 1, "eps"),
    (dict(db=None), 1, "delta_bias is NULL"),
    (dict(p=FAKE + 4), 1, "partials is not 16-byte aligned"),
    (dict(ys=1284), 1, "16-byte aligned"),
    (dict(xs=1272), 1, "shorter than the rows"),
    (dict(ys=1272), 1, "shorter than the rows"),
])
def test_add_layernorm_partials_rejects_bad_arguments(lib, over, code, msg):
    assert call_add_ln_partials(lib, **over) == code
    assert msg in lib.wdrz_last_error().decode()


def test_add_layernorm_partials_zero_rows_is_a_no_op(lib):
    assert call_add_ln_partials(lib, rows=0, x=None, p=None, db=None, w=None, b=None, y=None) == 0
