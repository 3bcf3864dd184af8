"""ctypes binding of libwdrz_attn.so (the C ABI declared in include/wdrz_attn.h).

The library is loaded lazily and exactly once. There is no fallback: if the shared object is
missing or fails to load, every compute entry point raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

RELEASE_LIB_PATH = Path(__file__).resolve().parent / "libwdrz_attn.so"
DEBUG_LIB_PATH = Path(__file__).resolve().parent / "libwdrz_attn_debug.so"


def debug_mode() -> bool:
    """WDRZ_DEBUG=1: host-side checks of device metadata before every cached-attention call
    (the debug library and the Python checks; synchronous, so not for graph capture)."""
    return os.environ.get("WDRZ_DEBUG", "0") not in ("", "0")


LIB_PATH = DEBUG_LIB_PATH if debug_mode() else RELEASE_LIB_PATH

WDRZ_F32, WDRZ_F16, WDRZ_BF16 = 0, 1, 2
WDRZ_OK, WDRZ_EINVAL, WDRZ_EUNSUPPORTED, WDRZ_ELAUNCH, WDRZ_EWORKSPACE = 0, 1, 2, 3, 4

# Every symbol include/wdrz_attn.h declares (tests check the .so exports all of them).
EXPORTED_SYMBOLS = (
    "wdrz_last_error",
    "wdrz_abi_version",
    "wdrz_build_id",
    "wdrz_attn_fwd",
    "wdrz_attn_kvcache_workspace_size",
    "wdrz_attn_kvcache",
    "wdrz_attn_kvcache_noalloc",
    "wdrz_add_layernorm",
    "wdrz_masked_argmax",
    "wdrz_linear",
    "wdrz_linear_partials",
    "wdrz_add_layernorm_partials",
    "wdrz_log_mel_workspace_size",
    "wdrz_log_mel",
    "wdrz_dtw_qk",
    "wdrz_dtw_prep_workspace_size",
    "wdrz_dtw_prep",
    "wdrz_dtw_attention_prep",
    "wdrz_kv_fill",
    "wdrz_median_filter",
)
ABI_VERSION = 1

_lock = threading.Lock()
_lib = None
_load_error: str | None = None

_i64 = ctypes.c_int64
_p = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.c_void_p


def _declare(lib: ctypes.CDLL) -> None:
    lib.wdrz_last_error.restype = ctypes.c_char_p
    lib.wdrz_last_error.argtypes = []
    lib.wdrz_abi_version.restype = ctypes.c_int
    lib.wdrz_abi_version.argtypes = []
    lib.wdrz_attn_fwd.restype = ctypes.c_int
    lib.wdrz_attn_fwd.argtypes = [
        ctypes.c_int, _p, _p, _p, _p,  # dtype, q, k, v, o
        _i64, _i64, _i64, _i64, _i64,  # B, H, Lq, Lk, D
        _i64p, _i64p, _i64p, _i64p,  # strides
        ctypes.c_float, ctypes.c_int, _p,  # scale, causal, stream
    ]
    lib.wdrz_attn_kvcache_workspace_size.restype = ctypes.c_size_t
    lib.wdrz_attn_kvcache_workspace_size.argtypes = [_i64, _i64, _i64, _i64, _i64]
    lib.wdrz_attn_kvcache.restype = ctypes.c_int
    lib.wdrz_attn_kvcache.argtypes = [
        ctypes.c_int, _p, _p, _p, _p, _p,  # dtype, q, k_cache, v_cache, k_new, v_new
        _i32p, _i32p, _p,  # cache_seqlens, cache_batch_idx, out
        _i64, _i64, _i64, _i64, _i64, _i64,  # B, sq, H, D, n_slots, Lmax
        _i64p, _i64p, _i64p, _i64p, _i64p, _i64p,  # strides
        ctypes.c_float, ctypes.c_int,  # softmax_scale, causal
        _p, ctypes.c_size_t, _p,  # workspace, bytes, stream
    ]
    lib.wdrz_attn_kvcache_noalloc.restype = ctypes.c_int
    lib.wdrz_attn_kvcache_noalloc.argtypes = lib.wdrz_attn_kvcache.argtypes[:-3] + [_p]  # no workspace
    lib.wdrz_add_layernorm.restype = ctypes.c_int
    lib.wdrz_add_layernorm.argtypes = [
        ctypes.c_int, _p, _i64, _p, _i64,  # dtype, x, x stride, delta, delta stride
        _p, _p, _p, _i64, _i64, _i64,  # weight, bias, y, y stride, rows, n
        ctypes.c_float, _p,  # eps, stream
    ]
    lib.wdrz_linear.restype = ctypes.c_int
    lib.wdrz_linear.argtypes = [
        ctypes.c_int, _p, _i64, _p, _i64, _p,  # dtype, x, x stride, w, w stride, bias
        _p, _i64, _i64, _i64, _i64, ctypes.c_int, _p,  # y, y stride, M, N, K, activation, stream
    ]
    lib.wdrz_linear_partials.restype = ctypes.c_int
    lib.wdrz_linear_partials.argtypes = [
        ctypes.c_int, _p, _i64, _p, _i64, _p,  # dtype, x, x stride, w, w stride, partials
        _i64, _i64, _i64, ctypes.c_int, _p,  # M, N, K, n_split, stream
    ]
    lib.wdrz_add_layernorm_partials.restype = ctypes.c_int
    lib.wdrz_add_layernorm_partials.argtypes = [
        ctypes.c_int, _p, _i64, _p, ctypes.c_int, _p,  # dtype, x, x stride, partials, n_split, delta bias
        _p, _p, _p, _i64, _i64, _i64,  # weight, bias, y, y stride, rows, n
        ctypes.c_float, _p,  # eps, stream
    ]
    lib.wdrz_masked_argmax.restype = ctypes.c_int
    lib.wdrz_masked_argmax.argtypes = [
        ctypes.c_int, _p, _i64, _p, _i64, _p, _i64,  # dtype, logits, stride, blocked, stride, penalty, stride
        _p, _i64, _i64, _p,  # out, rows, V, stream
    ]
    lib.wdrz_log_mel_workspace_size.restype = ctypes.c_size_t
    lib.wdrz_log_mel_workspace_size.argtypes = [_i64, _i64]
    lib.wdrz_log_mel.restype = ctypes.c_int
    lib.wdrz_log_mel.argtypes = [
        _p, _i64, _i64, _i64, _p, _i64p,  # audio, B, n_samples, audio_stride, out, out strides
        _i64, _i64, _p, ctypes.c_size_t, _p,  # n_mels, out_frames, workspace, bytes, stream
    ]
    lib.wdrz_dtw_qk.restype = ctypes.c_int
    lib.wdrz_dtw_qk.argtypes = [
        ctypes.c_int, _p, _i64p, _p, _i64p,  # dtype, q_heads (host array), q strides, k_heads, k strides
        _p, _i64p,  # out, out strides
        _i64, _i64, _i64, _i64, _i64,  # B, H, T, A, D
        ctypes.c_float, _p,  # scale, stream
    ]
    lib.wdrz_dtw_prep_workspace_size.restype = ctypes.c_size_t
    lib.wdrz_dtw_prep_workspace_size.argtypes = [_i64, _i64, _i64, _i64]
    lib.wdrz_dtw_prep.restype = ctypes.c_int
    lib.wdrz_dtw_prep.argtypes = [
        _p, _i64p, _i32p, _i32p, _p, _i64p,  # weights, strides, lens, caps, out, out strides
        _i64, _i64, _i64, _i64, _i64, ctypes.c_int,  # B, H, T, A, C, medfilt_width
        _p, ctypes.c_size_t, _p,  # workspace, bytes, stream
    ]
    lib.wdrz_dtw_attention_prep.restype = ctypes.c_int
    lib.wdrz_dtw_attention_prep.argtypes = [
        ctypes.c_int, _p, _i64p, _p, _i64p, ctypes.c_float,  # dtype, q_heads, q strides, k_heads, k strides, scale
        _i32p, _i32p, _p, _i64p,  # lens, caps, out, out strides
        _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_int,  # B, H, T, A, D, C, medfilt_width
        _p, ctypes.c_size_t, _p,  # workspace, bytes, stream
    ]

    lib.wdrz_build_id.restype = ctypes.c_char_p
    lib.wdrz_build_id.argtypes = []

    lib.wdrz_kv_fill.restype = ctypes.c_int
    lib.wdrz_kv_fill.argtypes = [
        ctypes.c_int, _p, _p, _i64p, _p, _p, _i64p, _p,  # dtype, k/v src, src strides, k/v cache, cache strides, slots
        _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p,  # B, T, H, D, n_slots, Lmax, start_pos, stream
    ]

    lib.wdrz_median_filter.restype = ctypes.c_int
    lib.wdrz_median_filter.argtypes = [_p, _i64, _p, _i64, _i64, _i64, ctypes.c_int, _p]


def load() -> ctypes.CDLL:
    """Return the loaded library, raising RuntimeError when it cannot be loaded."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            _load_error = (
                f"{LIB_PATH} is not built; run `python -m whisperdrz_amd.build` "
                "(or __graft_entry__.build())"
            )
            raise RuntimeError(_load_error)
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:  # pragma: no cover - depends on the environment
            _load_error = f"failed to load {LIB_PATH}: {exc}"
            raise RuntimeError(_load_error) from exc
        try:
            _declare(lib)
        except AttributeError as exc:  # a library built from older sources
            _load_error = f"{LIB_PATH} lacks {exc}; rebuild it (python -m whisperdrz_amd.build)"
            raise RuntimeError(_load_error) from exc
        if lib.wdrz_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"{LIB_PATH} has ABI {lib.wdrz_abi_version()}, expected {ABI_VERSION}; rebuild it"
            )
        # the library must have been built from the sources next to it
        from .build import source_hash

        built, tree = lib.wdrz_build_id().decode(), source_hash()
        if built != tree:
            _load_error = (f"{LIB_PATH} was built from other sources (build id {built}, tree {tree}); "
                           "rebuild it (python -m whisperdrz_amd.build)")
            raise RuntimeError(_load_error)
        _lib = lib
        return lib


def available() -> bool:
    try:
        load()
        return True
    except RuntimeError:
        return False


def last_error() -> str:
    return load().wdrz_last_error().decode()


def strides4(s) -> ctypes.Array:
    return (ctypes.c_int64 * 4)(*[int(x) for x in s])
