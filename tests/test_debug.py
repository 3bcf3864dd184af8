"""Opt-in debug checks and the torch A/B switch (host logic, no GPU needed)."""
import os
import subprocess
import sys
import warnings

import numpy as np
import pytest

from whisperdrz_amd.debug import check_kvcache_metadata

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _arr(*x):
    return np.array(x, dtype=np.int32)


def test_valid_metadata_passes_silently():
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        check_kvcache_metadata(_arr(0, 10, 447), _arr(2, 0, 1), 1, 3, 448, True)
        # same slot, disjoint regions [0, 5) and [5, 10)
        check_kvcache_metadata(_arr(0, 5), _arr(1, 1), 5, 2, 448, True)
        # identity slots, cross-attention (no append): lengths are not looked at
        check_kvcache_metadata(None, None, 1, 4, 1500, False)
        check_kvcache_metadata(_arr(-7, 9999), _arr(0, 3), 1, 4, 1500, False)


@pytest.mark.parametrize("slots", [(0, 3), (-1, 0)])
def test_slot_out_of_range_raises(slots):
    with pytest.raises(ValueError, match="outside \\[0, 3\\)"):
        check_kvcache_metadata(_arr(0, 0), _arr(*slots), 1, 3, 448, True)
    with pytest.raises(ValueError, match="slot"):
        check_kvcache_metadata(None, _arr(*slots), 1, 3, 448, False)


@pytest.mark.parametrize("cs,sq", [((444,), 5), ((-1,), 1), ((448,), 1)])
def test_append_outside_the_cache_raises(cs, sq):
    with pytest.raises(ValueError, match="outside the cache"):
        check_kvcache_metadata(_arr(*cs), _arr(0), sq, 1, 448, True)


def test_repeated_slots_are_valid():
    # the padded rows of a bucketed decode graph repeat an active slot, with its length or not:
    # the appends apply in batch order, as in the fallback (model.py:51-54)
    check_kvcache_metadata(_arr(7, 3, 7), _arr(2, 0, 2), 1, 3, 448, True)
    check_kvcache_metadata(_arr(10, 0, 12), _arr(4, 1, 4), 5, 5, 448, True)


def _run(env_extra, code):
    env = dict(os.environ)
    env.pop("WDRZ_FORCE_TORCH", None)
    env.pop("WDRZ_DEBUG", None)
    env.update(env_extra)
    out = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    return out.stdout.strip()


def test_force_torch_switches_the_probe_off():
    from whisperdrz_amd import _lib

    code = "import whisperdrz_amd as w; print(w.HAS_WDRZ, w.probe(), w.force_torch())"
    assert _run({"WDRZ_FORCE_TORCH": "1"}, code) == "False False True"
    expect = str(_lib.available())
    assert _run({}, code) == f"{expect} {expect} False"
    assert _run({"WDRZ_FORCE_TORCH": "0"}, code) == f"{expect} {expect} False"


def test_debug_mode_selects_the_checked_library():
    code = "from whisperdrz_amd import _lib; print(_lib.LIB_PATH.name, _lib.debug_mode())"
    assert _run({"WDRZ_DEBUG": "1"}, code) == "libwdrz_attn_debug.so True"
    assert _run({}, code) == "libwdrz_attn.so False"


def test_debug_library_exports_every_symbol():
    import ctypes

    from whisperdrz_amd import _lib

    if not _lib.DEBUG_LIB_PATH.exists():
        pytest.skip("libwdrz_attn_debug.so is not built")
    lib = ctypes.CDLL(str(_lib.DEBUG_LIB_PATH))
    _lib._declare(lib)  # raises AttributeError for a missing export
    assert lib.wdrz_abi_version() == _lib.ABI_VERSION
